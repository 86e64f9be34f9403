"""GPU parity of the individual kernels against the CPU oracle, through the C ABI.

Bar: bit-exact. Integer block sums are exact integers; every float the kernels
produce follows the oracle's fixed operation order, so values must be equal bit
for bit, not merely close.
"""
import math
import sys

import numpy as np
import pytest

import minfer
import oracle_lib as O

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(99)


def say(*a):
    print("[gpu-kernels]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as T
    if not T.cuda.is_available():
        pytest.skip("no GPU")
    return T


def rand_q4(rows, nb):
    blk = np.zeros((rows, nb, 18), np.uint8)
    d = np.abs(RNG.normal(0, 0.002, (rows, nb))).astype(np.float16)
    blk[:, :, :2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = RNG.integers(0, 256, (rows, nb, 16), dtype=np.uint8)
    return blk


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("n", [32, 1536, 8960, 11008])
def test_quant_bit_exact(torch, n):
    say("quant n=%d" % n)
    x = (RNG.standard_normal(n) * RNG.uniform(0.01, 5)).astype(np.float32)
    x[:32] = 0
    xq, xd, xs8 = (torch.zeros(n, dtype=torch.int8, device="cuda"), torch.zeros(n // 32, device="cuda"),
                   torch.zeros(n // 32, dtype=torch.int32, device="cuda"))
    minfer.quant_q8(dev(torch, x), xq, xd, xs8)
    torch.cuda.synchronize()
    rq, rd, rs = O.quant_q8(x)
    assert np.array_equal(xq.cpu().numpy(), rq)
    assert np.array_equal(xd.cpu().numpy().view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(xs8.cpu().numpy(), rs)


@pytest.mark.parametrize("rows,nb,cb", [(128, 48, 8), (64, 28, 4), (192, 280, 8)])
def test_block_isums_exact(torch, rows, nb, cb):
    say("isums rows=%d nb=%d cb=%d" % (rows, nb, cb))
    blk = rand_q4(rows, nb)
    x = RNG.standard_normal(nb * 32).astype(np.float32)
    xq, _, _ = O.quant_q8(x)
    packed = dev(torch, minfer.pack_q4(blk.reshape(-1), rows, nb, cb))
    isum = torch.zeros(rows * nb, dtype=torch.int32, device="cuda")
    minfer.q4_block_isums(packed, rows, nb, cb, dev(torch, xq), isum)
    torch.cuda.synchronize()
    got = isum.cpu().numpy().reshape(rows, nb)
    nib = np.concatenate([blk[:, :, 2:] & 15, blk[:, :, 2:] >> 4], axis=2).astype(np.int64)
    ref = (nib * xq.reshape(nb, 32).astype(np.int64)[None]).sum(2)
    assert np.array_equal(got, ref)


GEMV_SHAPES = [  # (rows, in, cb, ks): S15 QKV/O/gate-up/down, S05 cb=4, lm_head slice
    (2048, 1536, 8, 6), (1536, 1536, 8, 6), (17920, 1536, 8, 4), (1536, 8960, 8, 8),
    (1152, 896, 4, 7), (9728, 896, 4, 4), (896, 4864, 8, 8), (4096, 1536, 8, 1), (256, 2048, 8, 3),
    # launch shapes: waves looping over 18 chunks, 3 waves, a 70-chunk segment (one-wave loop)
    (1536, 8960, 8, 2), (640, 1536, 8, 2), (512, 8960, 4, 1),
    # the config-1 microbench's own launch shapes (bench.py gemv_microbench): one-chunk
    # segments on one wave each (qkv, o, gate/up at ks 6), down ks 10, the whole S15 lm_head
    # at ks 2 (4 waves per workgroup, 3-chunk segments) and at ks 1; cb 4 one-chunk segments
    (17920, 1536, 8, 6), (1536, 8960, 8, 10), (151936, 1536, 8, 2), (151936, 1536, 8, 1),
    (9728, 896, 4, 7),
]


@pytest.mark.parametrize("rows,n_in,cb,ks", GEMV_SHAPES)
def test_gemv_bit_exact(torch, rows, n_in, cb, ks):
    say("gemv %dx%d cb=%d ks=%d" % (rows, n_in, cb, ks))
    nb = n_in // 32
    blk = rand_q4(rows, nb)
    x = RNG.standard_normal(n_in).astype(np.float32)
    xq, xd, xs8 = O.quant_q8(x)
    packed = dev(torch, minfer.pack_q4(blk.reshape(-1), rows, nb, cb))
    part = torch.zeros(ks * rows, device="cuda")
    y = torch.zeros(rows, device="cuda")
    minfer.gemv_q4(packed, rows, nb, cb, ks, dev(torch, xq), dev(torch, xd), dev(torch, xs8), part, y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    flat = blk.reshape(rows, nb * 18)
    ref = np.array([O.row_dot(flat[r], nb, cb, ks, xq, xd, xs8) for r in range(rows)], np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("nh,nkv,hd,L", [(12, 2, 128, 1), (12, 2, 128, 64), (12, 2, 128, 65), (12, 2, 128, 300),
                                         (14, 2, 64, 200), (16, 2, 128, 1024), (4, 2, 64, 130),
                                         (14, 2, 64, 1100), (16, 2, 128, 2049), (8, 1, 128, 5000),
                                         (32, 4, 64, 32768), (24, 4, 128, 32700), (12, 2, 128, 33000)])
def test_attention_bit_exact(torch, nh, nkv, hd, L):
    """chunked attention vs the oracle's canonical order; the last three cases give
    items of all 8, of 3 and of 3 query heads of a kv head (the register-held record
    merges), the last with more splits (33) than those merges hold"""
    say("attention nh=%d nkv=%d hd=%d L=%d" % (nh, nkv, hd, L))
    ctx = L + 5
    q = RNG.standard_normal((nh, hd)).astype(np.float32)
    k16 = RNG.standard_normal((nkv, ctx, hd)).astype(np.float16)
    v16 = RNG.standard_normal((nkv, ctx, hd)).astype(np.float16)
    scale = np.float32(1.0) / np.float32(math.sqrt(hd))
    scratch = torch.zeros(minfer.attn_scratch_floats(nh, hd, L), device="cuda")
    out = torch.zeros(nh * hd, device="cuda")
    minfer.attn_decode(dev(torch, q), dev(torch, k16.view(np.int16)), dev(torch, v16.view(np.int16)), nh, nkv, hd,
                       L, ctx, float(scale), scratch, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(nh, hd)
    G = nh // nkv
    for h in range(nh):
        kf = np.ascontiguousarray(k16[h // G].astype(np.float32))
        vf = np.ascontiguousarray(v16[h // G].astype(np.float32))
        ref = O.attention_canon(np.ascontiguousarray(q[h]), kf.ravel(), vf.ravel(), L, hd, hd, float(scale))
        assert np.array_equal(got[h].view(np.uint32), ref.view(np.uint32)), h


def test_stream_read_runs(torch):
    say("stream read 256 MB")
    buf = torch.zeros(256 << 20, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    minfer.stream_read(buf, buf.numel(), sink)
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0


def attention_case(torch, nh, nkv, hd, L, scratch, rng):
    ctx = L + 3
    q = rng.standard_normal((nh, hd)).astype(np.float32)
    k16 = rng.standard_normal((nkv, ctx, hd)).astype(np.float16)
    v16 = rng.standard_normal((nkv, ctx, hd)).astype(np.float16)
    scale = np.float32(1.0) / np.float32(math.sqrt(hd))
    out = torch.zeros(nh * hd, device="cuda")
    minfer.attn_decode(dev(torch, q), dev(torch, k16.view(np.int16)), dev(torch, v16.view(np.int16)), nh, nkv, hd,
                       L, ctx, float(scale), scratch, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(nh, hd)
    G = nh // nkv
    for h in range(nh):
        kf = np.ascontiguousarray(k16[h // G].astype(np.float32))
        vf = np.ascontiguousarray(v16[h // G].astype(np.float32))
        ref = O.attention_canon(np.ascontiguousarray(q[h]), kf.ravel(), vf.ravel(), L, hd, hd, float(scale))
        assert np.array_equal(got[h].view(np.uint32), ref.view(np.uint32)), (nh, L, h)


def test_attention_scratch_reuse(torch):
    """one scratch buffer, NaN-filled once, through calls of different shapes: every
    record a call reads it wrote itself, so neither the initial contents nor an earlier
    call's records change the result"""
    rng = np.random.default_rng(5)
    scratch = torch.full((minfer.attn_scratch_floats(16, 128, 5000),), float("nan"), device="cuda")
    for nh, nkv, hd, L in [(12, 2, 128, 3000), (4, 2, 64, 100), (12, 2, 128, 3000), (16, 2, 128, 5000),
                           (14, 2, 64, 1100), (12, 2, 128, 64)]:
        say("scratch reuse nh=%d hd=%d L=%d" % (nh, hd, L))
        attention_case(torch, nh, nkv, hd, L, scratch, rng)


def rope_rows(x, pos0, base=1e6):
    """NEOX RoPE of rows x[t] at absolute positions pos0 + t (float64)"""
    hd = x.shape[-1]
    half = hd // 2
    inv = base ** (-np.arange(half, dtype=np.float64) * 2 / hd)
    ang = (pos0 + np.arange(x.shape[-2], dtype=np.float64))[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)


@pytest.mark.parametrize("L", [512, 4096, 16384, 24001, 32768])
def test_attention_depth_config3(torch, L):
    """config 3: S15 attention (12 query / 2 kv heads, head_dim 128), one query, an
    fp16 K/V cache N(0,1) with RoPE at absolute positions 0..L-1. Bit-exact against
    the oracle's canonical order (past 16 chunks a two-level merge), within 1e-3
    relative of an fp64 softmax. 24001 takes items of 2 query heads and ends in a
    one-position chunk; 32768 takes items of 3 heads."""
    nh, nkv, hd = 12, 2, 128
    say("attention at depth L=%d" % L)
    rng = np.random.default_rng(L)
    q = rope_rows(rng.standard_normal((nh, 1, hd)), L - 1)[:, 0].astype(np.float32)
    k16 = rope_rows(rng.standard_normal((nkv, L, hd)), 0).astype(np.float16)
    v16 = rng.standard_normal((nkv, L, hd)).astype(np.float16)
    scale = np.float32(1.0) / np.float32(math.sqrt(hd))
    scratch = torch.zeros(minfer.attn_scratch_floats(nh, hd, L), device="cuda")
    out = torch.zeros(nh * hd, device="cuda")
    minfer.attn_decode(dev(torch, q), dev(torch, k16.view(np.int16)), dev(torch, v16.view(np.int16)), nh, nkv, hd,
                       L, L, float(scale), scratch, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(nh, hd)
    G = nh // nkv
    for h in range(nh):
        kf = np.ascontiguousarray(k16[h // G].astype(np.float32))
        vf = np.ascontiguousarray(v16[h // G].astype(np.float32))
        ref = O.attention_canon(np.ascontiguousarray(q[h]), kf.ravel(), vf.ravel(), L, hd, hd, float(scale))
        assert np.array_equal(got[h].view(np.uint32), ref.view(np.uint32)), h
        sc = (kf.astype(np.float64) @ q[h].astype(np.float64)) * float(scale)
        p = np.exp(sc - sc.max())
        r64 = (p / p.sum()) @ vf.astype(np.float64)
        assert np.abs(got[h] - r64).max() <= 1e-3 * np.abs(r64).max(), h
