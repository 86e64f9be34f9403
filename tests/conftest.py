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


def gguf_tensor(path, name):
    """(ggml type, dims, file offset of the data) of a tensor of a GGUF v3 file"""
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
    align = [32]

    def skip(t, key=None):
        if t == 8:
            rstr()
        elif t == 9:
            et, n = rd("I"), rd("Q")
            for _ in range(n):
                skip(et)
        else:
            if key == "general.alignment":
                align[0] = struct.unpack_from("<I", b, o[0])[0]
            o[0] += sizes[t]

    assert b[:4] == b"GGUF" and rd("I") == 3
    nt, nkv = rd("Q"), rd("Q")
    for _ in range(nkv):
        k, t = rstr(), rd("I")
        skip(t, k)
    found = None
    for _ in range(nt):
        nm = rstr()
        nd = rd("I")
        dims = [rd("Q") for _ in range(nd)]
        ty, off = rd("I"), rd("Q")
        if nm == name:
            found = (ty, dims, off)
    base = (o[0] + align[0] - 1) // align[0] * align[0]
    if found is None:
        raise KeyError(name)
    return found[0], found[1], base + found[2]


def tie_head_gguf(src, dst, i, j, k, m):
    """A copy of the q4_0-headed GGUF src whose output.weight has exact argmax ties at
    every position: every row's block scales are zeroed except rows i, j, k, m; row j
    is a copy of row i, and rows k and m are row i with every block scale negated. The
    logits are then v, v, -v, -v at i, j, k, m (the same float operations, exactly
    negated) and 0 elsewhere: the greedy token is i when v > 0, k when v < 0, each with
    margin 0 (first max, cpu_infer.cpp:153-154)."""
    import numpy as np
    ty, dims, off = gguf_tensor(src, "output.weight")
    assert ty == 2, "the head must be q4_0"
    cols, rows = dims[0], dims[1]
    rb = cols // 32 * 18
    with open(src, "rb") as f:
        data = bytearray(f.read())
    w = np.frombuffer(data, dtype=np.uint8, count=rows * rb, offset=off).reshape(rows, rb).copy()
    blk = w.reshape(rows, cols // 32, 18)
    keep = blk[i].copy()
    blk[:, :, 0:2] = 0
    blk[i] = keep
    blk[j] = keep
    neg = keep.copy()
    neg[:, 1] ^= 0x80                      # fp16 sign bit of each block scale (little endian)
    blk[k] = neg
    blk[m] = neg
    data[off:off + rows * rb] = blk.reshape(-1).tobytes()
    with open(dst, "wb") as f:
        f.write(bytes(data))
    return dst
