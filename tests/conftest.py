import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "nano-inference_amd"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

TMP = os.environ.get("MI_TMP", os.path.join(os.environ.get("TMPDIR", "/tmp"), "mi"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on the CPU")


@pytest.fixture(scope="session")
def tmpdir_mi():
    os.makedirs(TMP, exist_ok=True)
    return TMP


def synth_cached(name, shape, seed, expect_hash=None):
    """Regenerate a synthetic GGUF (or reuse an identical one) under TMP."""
    import minfer
    os.makedirs(TMP, exist_ok=True)
    path = os.path.join(TMP, "%s-%d.gguf" % (name, seed))
    marker = path + ".ok"
    if not (os.path.exists(path) and os.path.exists(marker)):
        minfer.synth_gguf(path, shape, seed)
        open(marker, "w").close()
    return path
