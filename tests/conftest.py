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


def synth_cached(name, shape, seed, expect_hash=None, **types):
    """Regenerate a synthetic GGUF (or reuse an identical one) under TMP. types:
    emb_type / head_type / down_type / tied / qk_bias_std / norm_offset, as
    minfer.synth_gguf takes them."""
    import minfer
    os.makedirs(TMP, exist_ok=True)
    tag = "".join("-%s%s" % (k, "%g" % v) for k, v in sorted(types.items()))
    path = os.path.join(TMP, "%s-%d%s.gguf" % (name, seed, tag))
    marker = path + ".ok"
    if not (os.path.exists(path) and os.path.exists(marker)):
        minfer.synth_gguf(path, shape, seed, **types)
        open(marker, "w").close()
    return path
