"""The allocation-free attention entry point (mi_attn_decode_noalloc) against
mi_attn_decode with a caller-allocated workspace, through the C ABI.

Bar: bit-identical outputs (both run the same kernel over the same records), on
two calls in a row, the second with a smaller input, so the shared library-held
scratch is reused with the previous call's contents in it; a shape whose scratch
would exceed the library's fixed size is rejected with a clear error.
"""
import math
import sys

import numpy as np
import pytest

import minfer

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu-noalloc]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as T
    if not T.cuda.is_available():
        pytest.skip("no GPU")
    return T


def run_both(torch, rng, nh, nkv, hd, L):
    ctx = L + 3
    q = torch.from_numpy(rng.standard_normal((nh, hd)).astype(np.float32)).cuda()
    kc = torch.from_numpy(rng.standard_normal((nkv, ctx, hd)).astype(np.float16).view(np.int16)).cuda()
    vc = torch.from_numpy(rng.standard_normal((nkv, ctx, hd)).astype(np.float16).view(np.int16)).cuda()
    scale = float(np.float32(1.0) / np.float32(math.sqrt(hd)))
    scratch = torch.zeros(minfer.attn_scratch_floats(nh, hd, L), device="cuda")
    ref = torch.full((nh * hd,), float("nan"), device="cuda")
    got = torch.full((nh * hd,), float("nan"), device="cuda")
    minfer.attn_decode(q, kc, vc, nh, nkv, hd, L, ctx, scale, scratch, ref)
    minfer.attn_decode_noalloc(q, kc, vc, nh, nkv, hd, L, ctx, scale, got)
    torch.cuda.synchronize()
    return got.cpu().numpy(), ref.cpu().numpy()


@pytest.mark.parametrize("first,second", [((12, 2, 128, 32768), (12, 2, 128, 4000)),
                                          ((14, 2, 64, 20000), (4, 2, 64, 130))])
def test_noalloc_matches_workspace_entry(torch, first, second):
    rng = np.random.default_rng(first[3])
    for shape in (first, second):
        say("noalloc nh=%d nkv=%d hd=%d L=%d" % shape)
        got, ref = run_both(torch, rng, *shape)
        assert not np.isnan(ref).any()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), shape


def test_noalloc_rejects_oversize(torch):
    """a shape whose records exceed the fixed scratch: MI_ERR_SHAPE, nothing launched"""
    nh, hd = 32, 128
    L = 1 << 20
    assert minfer.attn_scratch_floats(nh, hd, L) > minfer.ATTN_NOALLOC_SCRATCH_FLOATS
    q = torch.zeros(nh * hd, device="cuda")
    kv = torch.zeros(8, dtype=torch.int16, device="cuda")
    out = torch.zeros(nh * hd, device="cuda")
    with pytest.raises(minfer.MinferError) as ei:
        minfer.attn_decode_noalloc(q, kv, kv, nh, 4, hd, L, L, 0.1, out)
    assert ei.value.code == -4 and "scratch" in str(ei.value)


def test_noalloc_graph_capture(torch):
    """mi_attn_decode_noalloc captured into a HIP graph (after one eager call on the
    device, which looks the scratch address up) and replayed three times, with other
    eager work on the same scratch between the replays: every replay equals the eager
    result bit for bit."""
    rng = np.random.default_rng(5)
    nh, nkv, hd, L = 12, 2, 128, 3000
    ctx = L + 3
    q = torch.from_numpy(rng.standard_normal((nh, hd)).astype(np.float32)).cuda()
    kc = torch.from_numpy(rng.standard_normal((nkv, ctx, hd)).astype(np.float16).view(np.int16)).cuda()
    vc = torch.from_numpy(rng.standard_normal((nkv, ctx, hd)).astype(np.float16).view(np.int16)).cuda()
    scale = float(np.float32(1.0) / np.float32(math.sqrt(hd)))
    eager = torch.full((nh * hd,), float("nan"), device="cuda")
    minfer.attn_decode_noalloc(q, kc, vc, nh, nkv, hd, L, ctx, scale, eager)
    torch.cuda.synchronize()
    want = eager.cpu().numpy()
    assert not np.isnan(want).any()
    out = torch.full((nh * hd,), float("nan"), device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):                 # captured on torch's capture stream (the current one)
        minfer.attn_decode_noalloc(q, kc, vc, nh, nkv, hd, L, ctx, scale, out)
    other = torch.empty((nh * hd,), device="cuda")
    for rep in range(3):
        say("noalloc graph replay %d" % rep)
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
        # eager work on the same scratch between replays (a smaller shape)
        minfer.attn_decode_noalloc(q[:4].contiguous(), kc, vc, 4, nkv, hd, 500, ctx, scale, other[:4 * hd])
        torch.cuda.synchronize()
