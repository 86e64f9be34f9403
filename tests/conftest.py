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


def gguf_kv_u32_offset(path, key):
    """file offset of a u32 metadata value of a GGUF v3 file"""
    import struct
    with open(path, "rb") as f:
        b = f.read()
    o = [4]

    def rd(fmt):
        v = struct.unpack_from("<" + fmt, b, o[0])[0]
        o[0] += struct.calcsize("<" + fmt)
        return v

    def rstr():
        n = rd("Q")
        o[0] += n
        return b[o[0] - n:o[0]].decode()

    sizes = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}

    def skip(t):
        if t == 8:
            rstr()
        elif t == 9:
            et, n = rd("I"), rd("Q")
            for _ in range(n):
                skip(et)
        else:
            o[0] += sizes[t]

    assert b[:4] == b"GGUF" and rd("I") == 3
    _, nkv = rd("Q"), rd("Q")
    for _ in range(nkv):
        k, t = rstr(), rd("I")
        if k == key:
            assert t == 4
            return o[0]
        skip(t)
    raise KeyError(key)
