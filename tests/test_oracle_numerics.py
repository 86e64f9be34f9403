"""Pins the oracle's scalar building blocks against mathematics and numpy.

Each check is chosen so that a plausible mistake in the oracle (wrong rounding
mode, swapped nibble order, dropped -8 term, wrong reduction, wrong exp range
reduction) fails it. None of these call the GPU.
"""
import math
import os

import numpy as np
import pytest

import oracle_lib as O

RNG = np.random.default_rng(1234)


def ulp_dist(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def test_f16_to_f32_all_patterns():
    L = O.lib()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isinf(got[np.isinf(ref)])) and np.all(np.isnan(got[np.isnan(ref)]))


def test_f32_to_f16_round_nearest_even():
    L = O.lib()
    x = np.concatenate([
        RNG.standard_normal(20000).astype(np.float32) * np.float32(2.0) ** RNG.integers(-30, 17, 20000).astype(np.float32),
        # exact ties between two halves: midpoints of consecutive fp16 values (normal and subnormal)
        ((np.arange(1, 2000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24)),
        ((np.arange(1024, 2047, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10)),
        np.array([65504.0, 65519.99, 65520.0, 1e9, -1e9, 0.0, -0.0, 2.0 ** -25, 2.0 ** -26], np.float32),
    ])
    ref = x.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, ref)


def test_expf_against_libm():
    xs = np.concatenate([np.linspace(-87.0, 88.7, 200001, dtype=np.float32),
                         RNG.uniform(-20, 20, 50000).astype(np.float32)])
    got = np.array([O.expf(float(v)) for v in xs], np.float32)
    ref = np.exp(xs.astype(np.float64)).astype(np.float32)
    assert ulp_dist(got, ref).max() <= 2
    assert O.expf(0.0) == 1.0
    assert O.expf(-87.5) == 0.0 and O.expf(-1000.0) == 0.0
    assert math.isinf(O.expf(89.0)) and O.expf(88.72) < math.inf
    assert math.isnan(O.expf(float("nan")))


def test_quant_q8_properties():
    x = (RNG.standard_normal(32 * 400) * np.repeat(RNG.uniform(0.01, 10, 400), 32)).astype(np.float32)
    x[:32] = 0.0                                     # all-zero block
    xq, xd, xs8 = O.quant_q8(x)
    blocks = x.reshape(-1, 32).astype(np.float64)
    q = xq.reshape(-1, 32).astype(np.int64)
    amax = np.abs(blocks).max(1)
    assert np.all(np.abs(q) <= 127)
    assert np.array_equal(xs8, 8 * q.sum(1))
    assert np.all(q[0] == 0) and xd[0] == 0.0
    nz = amax > 0
    # the largest element maps to +-127, scales are fp16(amax/127) (relative 2^-11)
    assert np.all(np.abs(q[nz]).max(1) == 127)
    assert np.all(np.abs(xd[nz] / (amax[nz] / 127.0) - 1) <= 2.0 ** -11 + 1e-7)
    # round to nearest: |x*127/amax - q| <= 1/2 (+ float slack)
    frac = np.abs(blocks[nz] * (127.0 / amax[nz])[:, None] - q[nz])
    assert frac.max() <= 0.5 + 1e-4


def test_quant_q8_ties_to_even():
    # amax 127 makes the scale exactly 1, so x = k + 0.5 is an exact tie
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 4.5]
    xq, xd, _ = O.quant_q8(x)
    assert xq[:9].tolist() == [127, 0, 2, 2, 0, -2, -2, 4, 4]
    assert xd[0] == 1.0


def make_block(d, nibbles):
    """q4_0 block bytes: fp16 d, byte j = nibble[j] | nibble[j+16] << 4 (gguf.h:94-101)."""
    n = np.asarray(nibbles, np.uint8)
    b = np.zeros(18, np.uint8)
    b[:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:] = n[:16] | (n[16:] << 4)
    return b


def test_q4_block_layout_known_answer():
    # byte 0 = 0x9F: element 0 is the low nibble (15 -> +7), element 16 the high (9 -> +1)
    blk = np.zeros(18, np.uint8)
    blk[:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2] = 0x9F
    blk[3:] = 0x88                                   # all other elements (8 - 8) = 0
    x = np.zeros(32, np.int8)
    x[0], x[16] = 3, 5
    isum = O.lib().orc_q4_block_isum(O.ptr(blk), O.ptr(x))
    # sum n_j x_j = 15*3 + 9*5 (+ 8*x of every other element that is zero)
    assert isum == 15 * 3 + 9 * 5


def test_q4_block_isum_all_pairs():
    # every nibble value against every int8 value, in every element position
    L = O.lib()
    xs = np.arange(-128, 128, dtype=np.int64)
    for pos in (0, 7, 15, 16, 23, 31):
        for nib in range(16):
            nibbles = np.full(32, 8, np.uint8)
            nibbles[pos] = nib
            blk = make_block(1.0, nibbles)
            for xv in xs[::5].tolist() + [-128, 127]:
                x = np.zeros(32, np.int8)
                x[pos] = xv
                x[(pos + 1) % 32] = 1
                got = L.orc_q4_block_isum(O.ptr(blk), O.ptr(x))
                assert got == nib * xv + 8 * 1


def test_q4_row_dot_matches_float64():
    nb = 48
    for cb, ks in [(8, 1), (8, 6), (4, 5), (8, 4)]:
        blocks = np.stack([make_block(abs(RNG.normal(0, 0.002)), RNG.integers(0, 16, 32)) for _ in range(nb)])
        x = RNG.standard_normal(nb * 32).astype(np.float32)
        xq, xd, xs8 = O.quant_q8(x)
        got = O.row_dot(blocks.reshape(-1), nb, cb, ks, xq, xd, xs8)
        # float64 reference from the dequantized block values and the int8 activations
        nib = np.concatenate([blocks[:, 2:] & 15, blocks[:, 2:] >> 4], axis=1).astype(np.float64)
        d = blocks[:, :2].copy().view(np.float16).astype(np.float64).ravel()
        terms = (d * xd.astype(np.float64))[:, None] * (nib - 8) * xq.reshape(nb, 32)
        ref = terms.sum()
        assert abs(got - ref) <= 1e-5 * np.abs(terms).sum(), (cb, ks, got, ref)


def test_rmsnorm_canon_matches_float64():
    for n in (896, 1536, 2048):
        x = RNG.standard_normal(n).astype(np.float32) * 3
        w = RNG.standard_normal(n).astype(np.float32) * 0.02
        got = O.rmsnorm_canon(x, w, 1e-6)
        xd = x.astype(np.float64)
        ref = xd / np.sqrt((xd * xd).mean() + 1e-6) * w
        assert np.abs(got - ref).max() <= 3e-6 * np.abs(ref).max()


def test_butterfly64_sum():
    v = RNG.standard_normal(64).astype(np.float32)
    got = O.lib().orc_butterfly64(O.ptr(v))
    assert abs(got - math.fsum(v.astype(np.float64))) <= 1e-5 * np.abs(v).sum()
    ones = np.ones(64, np.float32)
    assert O.lib().orc_butterfly64(O.ptr(ones)) == 64.0


@pytest.mark.parametrize("L", [1, 5, 63, 64, 65, 200, 700, 1024, 1025, 1088, 3000])
def test_attention_canon_matches_float64(L):
    hd = 128
    q = RNG.standard_normal(hd).astype(np.float32)
    k = RNG.standard_normal((L, hd)).astype(np.float32)
    v = RNG.standard_normal((L, hd)).astype(np.float32)
    scale = np.float32(1 / math.sqrt(hd))
    s = k.astype(np.float64) @ q.astype(np.float64) * float(scale)
    p = np.exp(s - s.max())
    ref = (p / p.sum()) @ v.astype(np.float64)
    got = O.attention_canon(q, k.ravel(), v.ravel(), L, hd, hd, float(scale))
    assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    got32 = O.attention_fp32(q, k.ravel(), v.ravel(), L, hd, hd, float(scale))
    assert np.abs(got32 - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("L,peak", [(1025, 1024), (2100, 40), (2100, 1500), (4096, 4095)])
def test_attention_canon_split_tree_peaked(L, peak):
    """past 16 chunks the records merge as a two-level tree: a sharp score peak in one
    split (first, middle or last, including a split of one position) must carry its
    weight through both levels; a dropped or misweighted split fails the fp64 check"""
    hd = 64
    q = RNG.standard_normal(hd).astype(np.float32)
    k = RNG.standard_normal((L, hd)).astype(np.float32) * 0.3
    k[peak] = q * (6.0 * math.sqrt(hd) / float(q @ q))      # score 6 against scores ~N(0, 0.3)
    v = RNG.standard_normal((L, hd)).astype(np.float32)
    scale = np.float32(1 / math.sqrt(hd))
    s = k.astype(np.float64) @ q.astype(np.float64) * float(scale)
    p = np.exp(s - s.max())
    ref = (p / p.sum()) @ v.astype(np.float64)
    assert p[peak] == 1.0 and 0.05 < 1 / p.sum() < 0.5   # the peak weighs, so do the others
    got = O.attention_canon(q, k.ravel(), v.ravel(), L, hd, hd, float(scale))
    assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


def test_rope_cs_float_theta():
    import ctypes as C
    c, s = C.c_float(), C.c_float()
    for pos in (0, 1, 17, 4095, 32767):
        for i in (0, 1, 31, 63):
            O.lib().orc_rope_cs(pos, i, 128, C.c_float(1e6), C.byref(c), C.byref(s))
            theta = np.float32(pos) * np.float32(np.float32(1e6) ** np.float32(np.float32(-2.0 * i) / np.float32(128)))
            assert abs(c.value - math.cos(float(theta))) <= 2e-7 and abs(s.value - math.sin(float(theta))) <= 2e-7
    O.lib().orc_rope_cs(0, 5, 128, C.c_float(1e6), C.byref(c), C.byref(s))
    assert c.value == 1.0 and s.value == 0.0


@pytest.mark.parametrize("hd", [64, 128])
def test_rope_rotate_known_answers(hd):
    """NEOX RoPE (cpu_infer.cpp:49-61) rotates pair (i, i + hd/2) counter-clockwise:
    a quarter turn (cos 0, sin 1) maps (x, y) to (-y, x), a half turn to (-x, -y), and
    no other element moves. A flipped sign gives (y, -x); adjacent pairs (2i, 2i+1),
    the GPT-J layout, move other elements."""
    rng = np.random.default_rng(hd)
    nh, half = 3, hd // 2
    v = rng.standard_normal(nh * hd).astype(np.float32)
    x, y = v.reshape(nh, hd)[:, :half], v.reshape(nh, hd)[:, half:]
    quarter = O.rope_rotate(v, nh, hd, np.zeros(half), np.ones(half)).reshape(nh, hd)
    assert np.array_equal(quarter[:, :half], -y) and np.array_equal(quarter[:, half:], x)
    halfturn = O.rope_rotate(v, nh, hd, -np.ones(half), np.zeros(half)).reshape(nh, hd)
    assert np.array_equal(halfturn, -v.reshape(nh, hd))
    # one pair at a quarter turn, the rest at angle 0: only that pair changes
    c, s = np.ones(half), np.zeros(half)
    c[5], s[5] = 0.0, 1.0
    one = O.rope_rotate(v, nh, hd, c, s).reshape(nh, hd)
    moved = np.argwhere(one != v.reshape(nh, hd))[:, 1]
    assert set(moved.tolist()) == {5, 5 + half}
    assert np.array_equal(one[:, 5], -y[:, 5]) and np.array_equal(one[:, 5 + half], x[:, 5])


@pytest.mark.parametrize("pos", [1, 7, 100, 1023, 32767])
def test_rope_matches_float64_rotation(pos):
    """both modes' RoPE against a float64 rotation by theta_i = pos * base^(-2i/hd):
    norms of every pair are kept, and q.k of two rotated vectors depends only on the
    position difference (the property attention relies on)"""
    hd, nh, base, half = 128, 2, 1e6, 64
    rng = np.random.default_rng(pos)
    v = rng.standard_normal(nh * hd).astype(np.float32)
    th = pos * base ** (-2.0 * np.arange(half) / hd)
    vv = v.astype(np.float64).reshape(nh, hd)
    ref = np.concatenate([vv[:, :half] * np.cos(th) - vv[:, half:] * np.sin(th),
                          vv[:, :half] * np.sin(th) + vv[:, half:] * np.cos(th)], axis=1)
    c, s = O.rope_cs(pos, hd, base)
    # float32 theta: |theta| <= pos, so its rounding error is ~pos * 6e-8
    tol = 1e-5 + pos * 2.4e-7
    for got in (O.rope_rotate(v, nh, hd, c, s), O.rope_fp32(v, nh, hd, pos, base)):
        got = got.astype(np.float64).reshape(nh, hd)
        assert np.abs(got - ref).max() <= tol * np.abs(vv).max()
        pn = lambda a: a[:, :half] ** 2 + a[:, half:] ** 2
        assert np.allclose(pn(got), pn(vv), rtol=1e-5, atol=1e-6)
    # relative position: rot(q, p+d) . rot(k, p) equals rot(q, d) . rot(k, 0)
    q, k = v[:hd], v[hd:]
    d = 5
    cq, sq = O.rope_cs(pos + d, hd, base)
    ck, sk = O.rope_cs(pos, hd, base)
    c0, s0 = O.rope_cs(d, hd, base)
    dot_far = float(np.dot(O.rope_rotate(q, 1, hd, cq, sq).astype(np.float64), O.rope_rotate(k, 1, hd, ck, sk)))
    dot_near = float(np.dot(O.rope_rotate(q, 1, hd, c0, s0).astype(np.float64), k.astype(np.float64)))
    assert abs(dot_far - dot_near) <= (1e-4 + pos * 5e-6) * np.linalg.norm(q) * np.linalg.norm(k)


class _Tensor(__import__("ctypes").Structure):
    import ctypes as C
    _fields_ = [("type", C.c_uint32), ("nd", C.c_int32), ("ne", C.c_int64 * 4), ("data", C.c_void_p)]


def _dequant(buf, type_, cols, rows=1, fma=False):
    import ctypes as C
    t = _Tensor(type_, 2, (C.c_int64 * 4)(cols, rows, 1, 1), buf.ctypes.data)
    out = np.zeros(cols * rows, np.float32)
    f = O.lib().orc_dequant_row_fma if fma else O.lib().orc_dequant_row
    for r in range(rows):
        f(C.addressof(t), r, out[r * cols:].ctypes.data)
    return out.reshape(rows, cols)


def _f16(x):
    return np.float16(x).view(np.uint16).tobytes()


def test_dequant_q8_0_codes_times_scale():
    rng = np.random.default_rng(41)
    codes = rng.integers(-128, 128, (3, 32), dtype=np.int8)
    ds = np.float16([0.5, -0.0078125, 3.25])
    buf = np.frombuffer(b"".join(_f16(d) + c.tobytes() for d, c in zip(ds, codes)), np.uint8).copy()
    got = _dequant(buf, 8, 96)[0]
    assert np.array_equal(got, (codes.astype(np.float32) * ds.astype(np.float32)[:, None]).ravel())


def test_dequant_q4_1_nibbles_scale_and_min():
    """GGUF q4_1: element j of a block in the low nibble of byte j, j + 16 in the high"""
    rng = np.random.default_rng(42)
    n = rng.integers(0, 16, (2, 32))
    d, m = np.float16([0.25, 1.5]), np.float16([-2.0, 0.125])
    packed = [(n[b, :16] | (n[b, 16:] << 4)).astype(np.uint8) for b in range(2)]
    buf = np.frombuffer(b"".join(_f16(d[b]) + _f16(m[b]) + packed[b].tobytes() for b in range(2)), np.uint8).copy()
    want = (n * d.astype(np.float32)[:, None] + m.astype(np.float32)[:, None]).astype(np.float32).ravel()
    # scales and mins chosen so that q*d + m is exact in fp32: fused or not, the same value
    assert np.array_equal(_dequant(buf, 3, 64)[0], want)
    assert np.array_equal(_dequant(buf, 3, 64, fma=True)[0], want)


def _q6k_encode(q, sc, d):
    """ggml's q6_K layout from its definition: 256 values as two halves of 128; in a
    half, value 32k + l (k = 0..3, l = 0..31) keeps its low 4 bits in ql[l + 32 (k & 1)]
    (low nibble for k < 2, high for k >= 2) and its high 2 bits in qh[l] bits 2k..2k+1;
    16 int8 scales (one per 16 values), fp16 d at the end"""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for half in range(2):
        for k in range(4):
            for l in range(32):
                v = int(q[128 * half + 32 * k + l])
                i = 64 * half + l + 32 * (k & 1)
                ql[i] |= (v & 15) << (4 * (k >= 2))
                qh[32 * half + l] |= (v >> 4) << (2 * k)
    return ql.tobytes() + qh.tobytes() + sc.astype(np.int8).tobytes() + _f16(d)


def test_dequant_q6_k_round_trip():
    rng = np.random.default_rng(43)
    q = rng.integers(0, 64, 512)
    sc = rng.integers(-64, 64, 32)
    d = np.float16([0.03125, 0.5])
    buf = np.frombuffer(_q6k_encode(q[:256], sc[:16], d[0]) + _q6k_encode(q[256:], sc[16:], d[1]), np.uint8).copy()
    assert buf.size == 420
    got = _dequant(buf, 14, 512)[0]
    grp = np.repeat(np.arange(32), 16)           # value i of superblock b uses scale 16 b + i // 16
    dd = np.repeat(d.astype(np.float32), 256)
    want = (dd * sc[grp].astype(np.float32)) * (q - 32).astype(np.float32)
    assert np.array_equal(got, want.astype(np.float32))


def test_requant_q4_0_recipe():
    """mega.cu:924-936: d = amax/7 stored as fp16, q = clamp(rint(y / d) + 8, 0, 15)
    with the unrounded 1/d; an all-zero block keeps d = 0 and codes 8"""
    y = np.zeros(64, np.float32)
    y[:32] = np.linspace(-3.5, 3.5, 32, dtype=np.float32)
    out = np.zeros(36, np.uint8)
    O.lib().orc_requant_q4_0_row(y.ctypes.data, 64, out.ctypes.data)
    d = np.frombuffer(out[:2].tobytes(), np.float16)[0]
    assert d == np.float16(np.float32(3.5) / np.float32(7))
    inv = np.float32(1) / (np.float32(3.5) / np.float32(7))
    q = np.clip(np.rint(y[:32] * inv).astype(int) + 8, 0, 15)
    assert np.array_equal(out[2:18], (q[:16] | (q[16:] << 4)).astype(np.uint8))
    assert np.frombuffer(out[18:20].tobytes(), np.float16)[0] == 0 and np.all(out[20:36] == 0x88)


def test_oracle_argmax_ties_take_the_first_row(tmpdir_mi):
    """Exact logit ties (output.weight rows i, j identical and k, m their negation, every
    other row zero, tests/conftest.py tie_head_gguf): at every position the greedy token
    is the first row of the winning pair, i (v > 0) or k (v < 0), with margin 0, in both
    oracle modes (cpu_infer.cpp:153-154 takes the first maximum)."""
    import minfer
    from conftest import synth_cached, tie_head_gguf
    shape = dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=4096)
    src = synth_cached("tie-src", shape, 31)
    path = tie_head_gguf(src, os.path.join(tmpdir_mi, "tie-31.gguf"), 100, 2000, 7, 3000)
    prompt = minfer.prompt_ids(4, 6, shape["n_vocab"])
    for mode in (O.MODE_FP32, O.MODE_Q8ACT):
        plan = O.Plan.make([8] * 5, [1, 1, 1, 2, 1]) if mode == O.MODE_Q8ACT else None
        m = O.Model(path, mode, plan=plan, max_seq=64)
        seen = set()
        for p, t in enumerate(prompt):
            a, mg, lg = m.forward(t, p, True)
            v = float(lg[100])
            assert lg[2000] == lg[100] and lg[7] == -lg[100] and lg[3000] == -lg[100]
            want = 100 if v > 0 else 7 if v < 0 else 0
            assert a == want and mg == 0.0, (mode, p, a, want, mg)
            seen.add(want)
        assert seen == {100, 7} or len(prompt) < 4, seen     # both signs occur over the prompt
