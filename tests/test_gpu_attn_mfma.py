"""GPU parity of the matrix-core attention (mi_attn_decode_mfma) through the C ABI.

Its chunk records come from fp16 MFMA contractions (q and the probabilities split
into two fp16 parts, K and V as stored), so it is not bit-identical to the canonical
order: the bar is the oracle's canonical result within 1e-5 relative (max |diff| /
max |ref|; the split keeps ~22 bits, so the measured error is ~1e-7) and, for config
3, an fp64 softmax within the 1e-3 relative that BASELINE config 3 states.
"""
import math
import sys

import numpy as np
import pytest

import minfer
import oracle_lib as O

pytestmark = pytest.mark.gpu

CANON_REL = 1e-5     # against the oracle's canonical fp32 order
F64_REL = 1e-3       # against an fp64 softmax (config 3's bar)


def say(*a):
    print("[gpu-attn-mfma]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as T
    if not T.cuda.is_available():
        pytest.skip("no GPU")
    return T


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_mfma(torch, q, k16, v16, nh, nkv, hd, L, ctx, scale, scratch=None):
    if scratch is None:
        scratch = torch.zeros(minfer.attn_scratch_floats(nh, hd, L), device="cuda")
    out = torch.zeros(nh * hd, device="cuda")
    minfer.attn_decode_mfma(dev(torch, q), dev(torch, k16.view(np.int16)), dev(torch, v16.view(np.int16)), nh, nkv,
                            hd, L, ctx, float(scale), scratch, out)
    torch.cuda.synchronize()
    return out.cpu().numpy().reshape(nh, hd)


def check_canon(got, q, k16, v16, nh, nkv, hd, L, scale, f64=False):
    G = nh // nkv
    worst = 0.0
    for h in range(nh):
        kf = np.ascontiguousarray(k16[h // G, :L].astype(np.float32))
        vf = np.ascontiguousarray(v16[h // G, :L].astype(np.float32))
        ref = O.attention_canon(np.ascontiguousarray(q[h]), kf.ravel(), vf.ravel(), L, hd, hd, float(scale))
        assert np.all(np.isfinite(got[h])), h
        rel = float(np.abs(got[h] - ref).max() / np.abs(ref).max())
        worst = max(worst, rel)
        assert rel <= CANON_REL, (h, rel)
        if f64:
            sc = (kf.astype(np.float64) @ q[h].astype(np.float64)) * float(scale)
            p = np.exp(sc - sc.max())
            r64 = (p / p.sum()) @ vf.astype(np.float64)
            assert np.abs(got[h] - r64).max() <= F64_REL * np.abs(r64).max(), h
    return worst


@pytest.mark.parametrize("nh,nkv,hd,L", [(12, 2, 128, 1), (12, 2, 128, 64), (12, 2, 128, 65), (12, 2, 128, 300),
                                         (14, 2, 64, 200), (16, 2, 128, 1024), (4, 2, 64, 130), (2, 2, 128, 77),
                                         (14, 2, 64, 1100), (16, 2, 128, 2049), (8, 1, 128, 5000),
                                         (32, 4, 64, 32768), (24, 4, 128, 32700), (12, 2, 128, 33000)])
def test_attention_mfma_vs_canon(torch, nh, nkv, hd, L):
    """every group size G = 1..8, both head sizes, ragged last chunks, one unit per
    workgroup and several (L = 32768: 1024 units on 512 workgroups)"""
    say("mfma attention nh=%d nkv=%d hd=%d L=%d" % (nh, nkv, hd, L))
    rng = np.random.default_rng(1000 + L + nh)
    ctx = L + 5
    q = rng.standard_normal((nh, hd)).astype(np.float32)
    k16 = rng.standard_normal((nkv, ctx, hd)).astype(np.float16)
    v16 = rng.standard_normal((nkv, ctx, hd)).astype(np.float16)
    scale = np.float32(1.0) / np.float32(math.sqrt(hd))
    got = run_mfma(torch, q, k16, v16, nh, nkv, hd, L, ctx, scale)
    worst = check_canon(got, q, k16, v16, nh, nkv, hd, L, scale)
    say("  max rel vs canonical %.2e" % worst)


@pytest.mark.parametrize("qscale", [1e-30, 1e-3, 30.0, 3e4])
def test_attention_mfma_q_range(torch, qscale):
    """q far from N(0,1): tiny (the power-of-two scaling keeps the fp16 parts normal),
    peaked softmax (30: scores ~ +-300), and beyond fp16 range (3e4 * N(0,1))"""
    nh, nkv, hd, L = 12, 2, 128, 700
    say("mfma attention q scale %g" % qscale)
    rng = np.random.default_rng(7)
    q = (rng.standard_normal((nh, hd)) * qscale).astype(np.float32)
    k16 = rng.standard_normal((nkv, L, hd)).astype(np.float16)
    v16 = rng.standard_normal((nkv, L, hd)).astype(np.float16)
    scale = np.float32(1.0) / np.float32(math.sqrt(hd))
    got = run_mfma(torch, q, k16, v16, nh, nkv, hd, L, L, scale)
    if qscale >= 30.0:
        # scores of hundreds: a score error of 1e-7 relative is ~1e-5 absolute, and the
        # probabilities move by that relative amount; still far inside the fp64 bar
        G = nh // nkv
        for h in range(nh):
            kf = k16[h // G].astype(np.float64)
            sc = (kf @ q[h].astype(np.float64)) * float(scale)
            p = np.exp(sc - sc.max())
            r64 = (p / p.sum()) @ v16[h // G].astype(np.float64)
            assert np.abs(got[h] - r64).max() <= F64_REL * np.abs(r64).max(), h
    else:
        check_canon(got, q, k16, v16, nh, nkv, hd, L, scale, f64=True)


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
def test_attention_mfma_config3(torch, L):
    """config 3 (12 query / 2 kv heads, head_dim 128, fp16 K/V N(0,1) with RoPE at
    absolute positions): within 1e-5 of the canonical order and 1e-3 of fp64"""
    nh, nkv, hd = 12, 2, 128
    say("mfma attention at depth L=%d" % L)
    rng = np.random.default_rng(L)
    q = rope_rows(rng.standard_normal((nh, 1, hd)), L - 1)[:, 0].astype(np.float32)
    k16 = rope_rows(rng.standard_normal((nkv, L, hd)), 0).astype(np.float16)
    v16 = rng.standard_normal((nkv, L, hd)).astype(np.float16)
    scale = np.float32(1.0) / np.float32(math.sqrt(hd))
    got = run_mfma(torch, q, k16, v16, nh, nkv, hd, L, L, scale)
    worst = check_canon(got, q, k16, v16, nh, nkv, hd, L, scale, f64=True)
    say("  max rel vs canonical %.2e" % worst)


def test_attention_mfma_scratch_reuse(torch):
    """a NaN-filled scratch shared by calls of different shapes, mixed with the
    canonical entry point: each call writes every record it reads"""
    rng = np.random.default_rng(11)
    scratch = torch.full((minfer.attn_scratch_floats(16, 128, 5000),), float("nan"), device="cuda")
    for nh, nkv, hd, L in [(12, 2, 128, 3000), (4, 2, 64, 100), (16, 2, 128, 5000), (12, 2, 128, 64)]:
        say("mfma scratch reuse nh=%d hd=%d L=%d" % (nh, hd, L))
        ctx = L + 3
        q = rng.standard_normal((nh, hd)).astype(np.float32)
        k16 = rng.standard_normal((nkv, ctx, hd)).astype(np.float16)
        v16 = rng.standard_normal((nkv, ctx, hd)).astype(np.float16)
        scale = np.float32(1.0) / np.float32(math.sqrt(hd))
        got = run_mfma(torch, q, k16, v16, nh, nkv, hd, L, ctx, scale, scratch)
        check_canon(got, q, k16, v16, nh, nkv, hd, L, scale)
        out = torch.zeros(nh * hd, device="cuda")
        minfer.attn_decode(dev(torch, q), dev(torch, k16.view(np.int16)), dev(torch, v16.view(np.int16)), nh, nkv, hd,
                           L, ctx, float(scale), scratch, out)
        torch.cuda.synchronize()
        canon = out.cpu().numpy().reshape(nh, hd)
        G = nh // nkv
        for h in range(nh):      # the canonical entry point on the same scratch: bit for bit
            kf = np.ascontiguousarray(k16[h // G, :L].astype(np.float32))
            vf = np.ascontiguousarray(v16[h // G, :L].astype(np.float32))
            ref = O.attention_canon(np.ascontiguousarray(q[h]), kf.ravel(), vf.ravel(), L, hd, hd, float(scale))
            assert np.array_equal(canon[h].view(np.uint32), ref.view(np.uint32)), (nh, hd, L, h)
