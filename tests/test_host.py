"""Host-side checks that need no GPU: the C ABI library loads and exports every
declared entry point, the q4_0 tile packing places every byte where the kernels
read it, the synthetic GGUF writer is deterministic and readable by the oracle's
independent GGUF reader, and errors are reported as codes, not exits."""
import os
import re

import numpy as np
import pytest

import minfer
import oracle_lib as O
from conftest import TMP

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "minfer.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", src))
    return sorted(n for n in names if n != "mi_token_cb")


def test_library_exports_every_declared_symbol():
    L = minfer.lib()
    names = declared_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(L, n), n
        assert n in minfer.SIGNATURES, "no ctypes signature for %s" % n


def test_q4_pack_layout():
    rng = np.random.default_rng(5)
    for rows, nb, cb in [(128, 48, 8), (64, 28, 4), (192, 16, 8)]:
        src = rng.integers(0, 256, rows * nb * 18, dtype=np.uint8)
        dst = minfer.pack_q4(src, rows, nb, cb)
        assert dst.size == rows * nb * 18 == minfer.packed_bytes(rows, nb, cb)
        blocks = src.reshape(rows, nb, 18)
        nc = nb // cb
        tiles = dst.reshape(rows // 64, nc, cb * 1152)
        for g in range(rows // 64):
            for c in range(nc):
                t = tiles[g, c]
                quants = t[:cb * 1024].reshape(cb, 64, 16)          # [block k][lane r][16 bytes]
                scales = t[cb * 1024:].reshape(64, cb, 2)           # [lane r][block k][fp16]
                ref = blocks[g * 64:(g + 1) * 64, c * cb:(c + 1) * cb]   # [r][k][18]
                assert np.array_equal(quants.transpose(1, 0, 2), ref[:, :, 2:])
                assert np.array_equal(scales, ref[:, :, :2])


def test_q4_pack_rejects_bad_shapes():
    assert minfer.packed_bytes(100, 48, 8) == 0      # rows not a multiple of 64
    assert minfer.packed_bytes(64, 28, 8) == 0       # blocks not a multiple of the chunk
    assert minfer.packed_bytes(64, 48, 6) == 0


def test_synth_deterministic_and_readable(tmp_path):
    shape = dict(n_layer=1, n_embd=128, n_ff=256, n_head=2, n_head_kv=1, n_vocab=512)
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    minfer.synth_gguf(a, shape, 11)
    minfer.synth_gguf(b, shape, 11)
    assert open(a, "rb").read() == open(b, "rb").read()
    minfer.synth_gguf(b, shape, 12)
    assert open(a, "rb").read() != open(b, "rb").read()
    m = O.Model(a, O.MODE_FP32, max_seq=8)
    c = m.cfg
    assert (c.n_layer, c.n_embd, c.n_ff, c.n_head, c.n_head_kv, c.head_dim, c.n_vocab) == (1, 128, 256, 2, 1, 64, 512)
    assert abs(c.rope_base - 1e6) < 1 and abs(c.rms_eps - 1e-6) < 1e-12
    tok, _ = m.forward(3, 0)
    assert 0 <= tok < 512


def test_synth_distributions(tmp_path):
    shape = dict(n_layer=1, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=1024)
    p = str(tmp_path / "d.gguf")
    minfer.synth_gguf(p, shape, 3)
    g = O.lib().orc_gguf_open(p.encode())
    assert g
    O.lib().orc_gguf_close(g)
    raw = open(p, "rb").read()
    # the fp32 embedding is the first tensor: N(0, 0.02)
    start = len(raw) - (1024 * 256 * 4 + 0)      # located via the oracle reader below instead
    del start
    m = O.Model(p, O.MODE_FP32, max_seq=4)
    assert m.cfg.n_vocab == 1024
    import ctypes as C
    L = O.lib()
    L.orc_gguf_tensor.restype = C.c_void_p
    L.orc_gguf_tensor.argtypes = [C.c_void_p, C.c_char_p]

    class T(C.Structure):
        _fields_ = [("type", C.c_uint32), ("nd", C.c_int32), ("ne", C.c_int64 * 4), ("data", C.c_void_p)]
    gg = L.orc_gguf_open(p.encode())
    te = T.from_address(L.orc_gguf_tensor(gg, b"token_embd.weight"))
    emb = np.ctypeslib.as_array((C.c_float * (1024 * 256)).from_address(te.data))
    assert abs(emb.mean()) < 1e-3 and abs(emb.std() - 0.02) < 1e-3
    tw = T.from_address(L.orc_gguf_tensor(gg, b"blk.0.ffn_up.weight"))
    nblk = 512 * 256 // 32
    blk = np.ctypeslib.as_array((C.c_uint8 * (nblk * 18)).from_address(tw.data)).reshape(nblk, 18)
    d = blk[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    assert np.all(d >= 0) and abs(d.mean() - 0.002 * np.sqrt(2 / np.pi)) < 1e-4
    nib = np.concatenate([blk[:, 2:] & 15, blk[:, 2:] >> 4]).ravel()
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.9 * counts.mean()
    L.orc_gguf_close(gg)


def test_prompt_ids_deterministic():
    a = minfer.prompt_ids(3, 64, 151936)
    assert a == minfer.prompt_ids(3, 64, 151936) and len(set(a)) > 60
    assert all(0 <= t < 151936 for t in a)
    assert minfer.prompt_ids(4, 64, 151936) != a


def test_oracle_gguf_errors(tmp_path):
    L = O.lib()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"NOPE" + b"\0" * 64)
    assert not L.orc_gguf_open(str(bad).encode())
    assert b"not a GGUF" in L.orc_gguf_error()
    trunc = tmp_path / "t.gguf"
    trunc.write_bytes(b"GGUF\x03\0\0\0" + b"\x05\0\0\0\0\0\0\0")
    assert not L.orc_gguf_open(str(trunc).encode())
    assert b"truncated" in L.orc_gguf_error()


def test_engine_load_reports_errors(tmp_path):
    n = C_int = None
    import ctypes as C
    cnt = C.c_int32()
    minfer.lib().mi_device_count(C.byref(cnt))
    with pytest.raises(minfer.MinferError) as ei:
        minfer.Engine(str(tmp_path / "missing.gguf"))
    if cnt.value == 0:
        assert ei.value.code == -5                   # no GPU here: a device error, not a crash
    else:
        assert ei.value.code == -3
    del n, C_int


def test_fnv1a64_published_vectors():
    """the FNV-1a 64 step (offset basis 14695981039346656037, prime 1099511628211):
    published test vectors of the FNV authors"""
    assert minfer.fnv1a64(b"") == 0xcbf29ce484222325
    assert minfer.fnv1a64(b"a") == 0xaf63dc4c8601ec8c
    assert minfer.fnv1a64(b"foobar") == 0x85944171f73967e8


def test_pred_hash_byte_layout():
    """mi_pred_hash = FNV-1a over (token, margin bits) little-endian per position from the
    reference's basis 1469598103934665603 (mega.cu:1197-1201); one changed margin bit or
    two swapped positions change it"""
    rng = np.random.default_rng(5)
    pred = rng.integers(0, 151936, 37).astype(np.int32)
    margin = rng.standard_normal(37).astype(np.float32)
    stream = np.stack([pred.astype("<i4").view("<u4"), margin.astype("<f4").view("<u4")], axis=1).tobytes()
    h = minfer.pred_hash(list(pred), list(margin))
    assert h == minfer.fnv1a64(stream, 1469598103934665603)
    assert minfer.pred_hash([], []) == 1469598103934665603
    m2 = margin.copy()
    m2.view(np.uint32)[3] ^= 1
    assert minfer.pred_hash(list(pred), list(m2)) != h
    p2 = pred.copy()
    p2[[4, 5]] = p2[[5, 4]]
    assert minfer.pred_hash(list(p2), list(margin)) != h


@pytest.mark.parametrize("name", ["mi_attn_decode", "mi_attn_decode_mfma"])
def test_attention_rejects_bad_shapes_before_any_launch(name):
    """the standalone attention entry points validate every argument before they
    touch the device: bad pointers and positions give MI_ERR_ARG (-1), shapes the
    kernels do not take give MI_ERR_SHAPE (-4); the pointers here are never
    dereferenced because every case is rejected first"""
    import ctypes as C
    fn = getattr(minfer.lib(), name)
    p = C.c_void_p(16)          # stand-in address: rejected calls never read it
    cases = [
        # (q, n_head, n_head_kv, hd, L, ctx, scratch, expected)
        (None, 12, 2, 128, 64, 64, p, -1),        # no q
        (p, 12, 2, 128, 64, 64, None, -1),        # no scratch
        (p, 12, 2, 128, 65, 64, p, -1),           # L > ctx
        (p, 12, 2, 128, 0, 64, p, -1),            # L < 1
        (p, 12, 5, 128, 64, 64, p, -4),           # n_head not a multiple of n_head_kv
        (p, 18, 2, 128, 64, 64, p, -4),           # 9 query heads per kv head
        (p, 12, 2, 96, 64, 64, p, -4),            # head_dim 96
        (p, 12, 2, 128, 600000, 600000, p, -4),   # more than 512 splits of 16 chunks
    ]
    for q, nh, nkv, hd, L, ctx, scr, want in cases:
        rc = fn(q, p, p, nh, nkv, hd, L, ctx, C.c_float(0.1), scr, p, None)
        assert rc == want, (name, nh, nkv, hd, L, ctx, rc)


LAYOUT_SHAPES = {
    "TINY": dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=4096),
    "SMALL": dict(n_layer=3, n_embd=512, n_ff=1536, n_head=8, n_head_kv=2, n_vocab=8192),
    "S05": "S05", "S15": "S15", "S3": "S3",
}


@pytest.mark.parametrize("name,max_ctx", [("TINY", 64), ("SMALL", 104), ("SMALL", 1100), ("S05", 160), ("S15", 208),
                                          ("S15", 4096), ("S3", 1040), ("S3", 1100)])
def test_step_indices_stay_inside_their_buffers(name, max_ctx):
    """Every index the single-token step and the multi-token phase bodies form (mi_check_layout,
    a host-side walk with each body's loop bounds over the shared layout functions) lies inside
    the buffer the engine allocates, for T = 1..8 at the first positions, across the first
    chunk boundaries, and at the end of the context. Cases: the CLI's 40-token prefill with 48
    generated (max_ctx 104), config 0/2 contexts, config 4 (S3 at context 1024), and a context
    past the two-level merge."""
    shape = LAYOUT_SHAPES[name]
    for n_cu in (256, 80):
        for T in range(1, 9):
            for pos in sorted({0, 1, 7, 8, 40, 63, 64, 65, max_ctx // 2, max_ctx - T - 1, max_ctx - T}):
                if pos < 0 or pos + T > max_ctx:
                    continue
                rc, msg = minfer.check_layout(shape, max_ctx, n_cu, T, pos)
                assert rc == 0, (name, max_ctx, n_cu, T, pos, msg)
    # a step past the context is refused, not walked
    rc, msg = minfer.check_layout(shape, max_ctx, 256, 8, max_ctx - 7)
    assert rc != 0 and "past the context" in msg

