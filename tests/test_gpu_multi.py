"""GPU parity of the multi-token (verify) step: T tokens at positions pos..pos+T-1
in one pass over the weights through int8 MFMA tiles (mi_step with T > 1).

Bar (the reference's own exactness check, mega.cu:1198-1204, is a hash of the
logits across T): every token's logits are bit-identical to running the same
tokens one at a time with T = 1, which is itself bit-identical to the q8act
oracle (test_gpu_engine.py); one case is also checked against the oracle directly.
Cases cover both chunk sizes of the q4 tiles (cb 8 and cb 4), a step that crosses
a 64-position attention chunk, and a context past the inline chunk merge. Each runs
the multi-token step both ways: as one launch per phase (persistent=1, the default)
and as one persistent launch with grid barriers between the phases (persistent=2).

Speculative generation (n-gram drafts verified by these steps) must be lossless:
its tokens and margins equal the plain greedy decode (tools/specbench.sh:36 checks
the same invariant on the reference).
"""
import sys

import numpy as np
import pytest

import minfer
import oracle_lib as O
from conftest import synth_cached

pytestmark = pytest.mark.gpu
TINY = dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=4096)
SMALL = dict(n_layer=3, n_embd=512, n_ff=1536, n_head=8, n_head_kv=2, n_vocab=8192)


def say(*a):
    print("[gpu-multi]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


MULTI = pytest.mark.parametrize("persistent", [1, 2], ids=["multi-phases", "multi-persistent"])


def multi_vs_single(eng, prompt, pos, T, seed, V):
    """prefill prompt[:pos], then one T-token step vs T single steps, same tokens"""
    eng.prefill(prompt[:pos])
    toks = minfer.prompt_ids(seed, T, V)
    am, mg, lg = eng.step(toks, pos, want_logits=True)
    for t in range(T):
        a, m, l1 = eng.step(toks[t], pos + t, want_logits=True)
        assert np.array_equal(bits(lg[t]), bits(l1)), "token %d of %d at pos %d: logits differ" % (t, T, pos)
        assert am[t] == a and bits(mg[t]) == bits(m)
    return toks, lg


@MULTI
@pytest.mark.parametrize("pos,T", [(12, 2), (12, 5), (61, 8), (3, 8)])
def test_tiny_multi_bit_identical(pos, T, persistent):
    path = synth_cached("eng-256", TINY, 7)
    say("tiny pos %d T %d persistent %d" % (pos, T, persistent))
    eng = minfer.Engine(path, max_ctx=256, persistent=persistent)
    prompt = minfer.prompt_ids(11, pos, TINY["n_vocab"])
    multi_vs_single(eng, prompt, pos, T, 100 + pos + T, TINY["n_vocab"])
    eng.close()


@MULTI
def test_small_multi_bit_identical_and_oracle(persistent):
    path = synth_cached("eng-512", SMALL, 21)
    pos, T = 70, 8
    say("small pos %d T %d (+ oracle) persistent %d" % (pos, T, persistent))
    eng = minfer.Engine(path, max_ctx=256, persistent=persistent)
    prompt = minfer.prompt_ids(12, pos, SMALL["n_vocab"])
    toks, lg = multi_vs_single(eng, prompt, pos, T, 5, SMALL["n_vocab"])
    p = eng.plan
    eng.close()
    orc = O.Model(path, O.MODE_Q8ACT, plan=O.Plan.make(p["cb"], p["ks"], p["attn_chunk"], p["kv_f16"]), max_seq=256)
    for i, tok in enumerate(list(prompt) + list(toks)):
        _, _, lo = orc.forward(tok, i, True)
        if i >= pos:
            assert np.array_equal(bits(lo), bits(lg[i - pos])), "oracle differs at pos %d" % i


@MULTI
def test_config0_multi_cb4_bit_identical(persistent):
    """S05 (hidden 896): q4 chunks of 4 blocks in the E-row matrices, head_dim 64"""
    shape = minfer.SHAPES["S05"]
    path = synth_cached("config0", shape, minfer.CONFIGS["config0"][1])
    say("config0 pos 16 T 8 persistent %d" % persistent)
    eng = minfer.Engine(path, max_ctx=64, persistent=persistent)
    assert eng.plan["cb"][0] == 4
    prompt = minfer.prompt_ids(minfer.CONFIGS["config0"][2], 16, shape["n_vocab"])
    multi_vs_single(eng, prompt, 16, 8, 17, shape["n_vocab"])
    eng.close()


@MULTI
def test_config2_multi_bit_identical(persistent):
    """S15: head_dim 128, the down matrix split into 10 K segments"""
    shape = minfer.SHAPES["S15"]
    path = synth_cached("config2", shape, minfer.CONFIGS["config2"][1])
    say("config2 pos 64 T 8 persistent %d" % persistent)
    eng = minfer.Engine(path, max_ctx=128, persistent=persistent)
    prompt = minfer.prompt_ids(minfer.CONFIGS["config2"][2], 64, shape["n_vocab"])
    multi_vs_single(eng, prompt, 64, 8, 19, shape["n_vocab"])
    eng.close()


@MULTI
@pytest.mark.parametrize("pos,T", [(1000, 6), (1020, 8)])
def test_long_context_multi_merge_phase(pos, T, persistent):
    """past 4 chunks the chunk records are merged by their own kernel, past 16 as a
    two-level tree (1020 + 8: the step's tokens see 16 and 17 chunks)"""
    path = synth_cached("eng-256", TINY, 7)
    say("tiny long context pos %d T %d persistent %d" % (pos, T, persistent))
    eng = minfer.Engine(path, max_ctx=1100, persistent=persistent)
    prompt = minfer.prompt_ids(13, pos, TINY["n_vocab"])
    multi_vs_single(eng, prompt, pos, T, 23, TINY["n_vocab"])
    eng.close()


@MULTI
def test_long_context_multi_merge_bounds(persistent):
    """2044 + 8: tokens 0-3 see 32 chunks (the most the multi-token merge takes with
    every record load issued first) and tokens 4-7 see 33 (past it, the split-by-split
    merge); T = 8 against eight single steps"""
    path = synth_cached("eng-256", TINY, 7)
    say("tiny long context pos 2044 T 8 persistent %d" % persistent)
    eng = minfer.Engine(path, max_ctx=2100, persistent=persistent)
    prompt = minfer.prompt_ids(14, 2044, TINY["n_vocab"])
    multi_vs_single(eng, prompt, 2044, 8, 31, TINY["n_vocab"])
    eng.close()


@MULTI
def test_long_context_multi_hd128(persistent):
    """head_dim 128 at context 1020 + 8 (16 and 17 chunks: the merge tree) on the
    attention-sensitive model (O(1) scores): T = 8 against eight single steps"""
    import json, os
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cpu_infer_attn.json")) as f:
        fx = json.load(f)
    path = synth_cached(fx["config"], fx["shape"], fx["model_seed"], **fx["types"])
    V = fx["shape"]["n_vocab"]
    say("hd128 long context pos 1020 T 8 persistent %d" % persistent)
    eng = minfer.Engine(path, max_ctx=1100, persistent=persistent)
    prompt = minfer.prompt_ids(43, 1020, V)
    multi_vs_single(eng, prompt, 1020, 8, 29, V)
    eng.close()


@MULTI
def test_config4_verify_step_bit_identical(persistent):
    """BASELINE config 4 at its own workload: S3 (hidden 2048, 36 layers, 16/2 heads,
    FF 11008), a 1024-token context, one 8-token verify step (the current token + 7
    drafts, TMAX = 8, mega.cu:50) bit-identical to the 8 tokens stepped one at a time"""
    name = "config4"
    cfg = minfer.CONFIGS[name]
    shape = minfer.SHAPES[cfg[0]]
    path = synth_cached(name, shape, cfg[1])
    say("config4 (S3) context 1024 T 8 persistent %d" % persistent)
    eng = minfer.Engine(path, max_ctx=cfg[3] + 16, persistent=persistent)
    prompt = minfer.prompt_ids(cfg[2], cfg[3], shape["n_vocab"])
    multi_vs_single(eng, prompt, cfg[3], 8, cfg[2] + 1, shape["n_vocab"])
    eng.close()


def test_config4_short_context_oracle():
    """S3 against the q8act oracle at a short context: an 8-token prompt stepped one
    at a time, then an 8-token step, every position's logits bit for bit"""
    cfg = minfer.CONFIGS["config4"]
    shape = minfer.SHAPES[cfg[0]]
    path = synth_cached("config4", shape, cfg[1])
    say("config4 (S3) pos 8 T 8 + oracle")
    eng = minfer.Engine(path, max_ctx=64)
    prompt = minfer.prompt_ids(cfg[2] + 2, 8, shape["n_vocab"])
    toks, lg = multi_vs_single(eng, prompt, 8, 8, cfg[2] + 3, shape["n_vocab"])
    p = eng.plan
    eng.close()
    orc = O.Model(path, O.MODE_Q8ACT, plan=O.Plan.make(p["cb"], p["ks"], p["attn_chunk"], p["kv_f16"]), max_seq=64)
    for i, tok in enumerate(list(prompt) + list(toks)):
        _, _, lo = orc.forward(tok, i, True)
        if i >= 8:
            assert np.array_equal(bits(lo), bits(lg[i - 8])), "oracle differs at pos %d" % i


@MULTI
def test_graph_replays_equal_direct_launches(persistent):
    """The multi-token step replays one captured HIP graph per (T, logits) with the
    position read from device memory. Replays at several positions, with eager
    single-token steps and host synchronizations in between, equal the same steps
    launched kernel by kernel, bit for bit, on every replay."""
    path = synth_cached("eng-512", SMALL, 21)
    V = SMALL["n_vocab"]
    prompt = minfer.prompt_ids(5, 100, V)
    g = minfer.Engine(path, max_ctx=256, graphs=1, persistent=persistent)
    d = minfer.Engine(path, max_ctx=256, graphs=0, persistent=1)
    for e in (g, d):
        e.prefill(prompt)            # 12 replays of the T=8 graph and one of T=4 in g
    cases = [(100, 8, True), (100, 8, False), (64, 5, True), (69, 8, True), (60, 8, False), (68, 2, True),
             (70, 8, True), (70, 8, True)]
    for i, (pos, T, want) in enumerate(cases):
        say("graph replay %d: pos %d T %d logits %d" % (i, pos, T, want))
        toks = minfer.prompt_ids(300 + i, T, V)
        rg = g.step(toks, pos, want_logits=want)
        rd = d.step(toks, pos, want_logits=want)
        assert rg[0] == rd[0] and np.array_equal(bits(rg[1]), bits(rd[1])), "replay %d: predictions differ" % i
        if want:
            assert np.array_equal(bits(rg[2]), bits(rd[2])), "replay %d: logits differ" % i
        a1 = g.step(toks[-1], pos + T)    # eager work between replays
        a2 = d.step(toks[-1], pos + T)
        assert a1[0] == a2[0] and bits(a1[1]) == bits(a2[1])
    g.close()
    d.close()


def test_multi_step_rejects_bad_T():
    path = synth_cached("eng-256", TINY, 7)
    eng = minfer.Engine(path, max_ctx=64)
    eng.prefill([1, 2, 3])
    with pytest.raises(minfer.MinferError):
        eng.step(list(range(9)), 3)
    eng.close()


def spec_vs_plain(path, prompt, n_gen, max_ctx):
    res = {}
    for spec in (0, 1):
        eng = minfer.Engine(path, max_ctx=max_ctx, spec=spec)
        eng.prefill(prompt)
        seen = []
        toks, margins = eng.generate(n_gen, callback=lambda t: seen.append(t) and False)
        assert seen == toks, "spec=%d: the callback saw %d of %d tokens" % (spec, len(seen), len(toks))
        res[spec] = (toks, margins, eng.stats())
        eng.close()
    (pt, pm, _), (st, sm, ss) = res[0], res[1]
    assert st == pt, "speculative output differs from plain greedy at %d" % next(
        i for i, (a, b) in enumerate(zip(st, pt)) if a != b)
    assert np.array_equal(bits(sm), bits(pm))
    return ss


@pytest.mark.parametrize("name", ["config0", "config2"])
def test_spec_generate_equals_plain(name):
    cfg = minfer.CONFIGS[name]
    shape = minfer.SHAPES[cfg[0]]
    path = synth_cached(name, shape, cfg[1])
    prompt = minfer.prompt_ids(cfg[2], cfg[3], shape["n_vocab"])
    st = spec_vs_plain(path, prompt, 128, cfg[3] + 160)
    say("%s speculative: %d verify steps for %d tokens, %d drafted, %d accepted" %
        (name, st["steps"], st["tokens"], st["drafted"], st["accepted"]))
    assert st["tokens"] == 128 and st["steps"] <= 128


def test_spec_generate_repetitive_prompt():
    """a prompt that repeats a 12-token pattern: the drafter proposes from the start"""
    path = synth_cached("eng-512", SMALL, 21)
    pattern = minfer.prompt_ids(31, 12, SMALL["n_vocab"])
    st = spec_vs_plain(path, pattern * 6, 96, 200)
    say("repetitive prompt: %d verify steps for %d tokens, %d drafted, %d accepted" %
        (st["steps"], st["tokens"], st["drafted"], st["accepted"]))
    assert st["drafted"] > 0


@pytest.mark.parametrize("case", ["config2", "repetitive", "config4"])
def test_spec_driven_on_device_equals_host_loop(case):
    """persistent = 2 and no callback: the speculative loop runs on the device (each
    persistent verify launch commits and drafts the next step itself). Tokens and margins
    equal the plain greedy decode, and the verify steps, drafts and acceptances equal the
    host-driven loop's one for one (the same draft rule in the same float arithmetic).
    config4: the drafter on its own shape (S3, the verify steps' int8 MFMA tiles at
    context ~1000): a synthetic repetitive stream of 1,000 tokens (a seeded 40-token
    pattern, 25 times) as the prompt, 64 generated."""
    if case == "config4":
        cfg = minfer.CONFIGS["config4"]
        shape = minfer.SHAPES[cfg[0]]
        path = synth_cached("config4", shape, cfg[1])
        prompt, n_gen = minfer.prompt_ids(cfg[2], 40, shape["n_vocab"]) * 25, 64
        max_ctx = len(prompt) + n_gen + 16
    elif case == "config2":
        cfg = minfer.CONFIGS["config2"]
        shape = minfer.SHAPES[cfg[0]]
        path = synth_cached("config2", shape, cfg[1])
        prompt, n_gen, max_ctx = minfer.prompt_ids(cfg[2], cfg[3], shape["n_vocab"]), 128, cfg[3] + 160
    else:
        path = synth_cached("eng-512", SMALL, 21)
        prompt, n_gen, max_ctx = minfer.prompt_ids(31, 12, SMALL["n_vocab"]) * 6, 96, 200
    res = {}
    for mode, opts in (("plain", dict(spec=0)), ("host", dict(spec=1, persistent=1)),
                       ("host_persistent", dict(spec=1, persistent=2)), ("device", dict(spec=2, persistent=2))):
        say("%s: %s" % (case, mode))
        eng = minfer.Engine(path, max_ctx=max_ctx, **opts)
        eng.prefill(prompt)
        toks, margins = eng.generate(n_gen)
        res[mode] = (toks, margins, eng.stats())
        eng.close()
    for mode in ("host", "host_persistent", "device"):
        assert res[mode][0] == res["plain"][0], mode
        assert np.array_equal(bits(res[mode][1]), bits(res["plain"][1])), mode
    h, d = res["host"][2], res["device"][2]
    say("%s: %d steps, %d drafted, %d accepted (device %.1f ms, host loop %.1f ms)" %
        (case, d["steps"], d["drafted"], d["accepted"], d["decode_ms"], h["decode_ms"]))
    for k in ("steps", "tokens", "drafted", "accepted"):
        assert d[k] == h[k] == res["host_persistent"][2][k], (k, d[k], h[k])


def test_spec_driven_on_device_stops_at_eos(tmp_path):
    """An eos stop inside a verify step's accepted run, with the commit on the device:
    the output ends at the eos exactly as the plain decode's does (mega.cu:1014-1017
    stops at tokenizer.ggml.eos_token_id), and a step at the eos position afterwards
    gives the plain engine's logits bit for bit (the drafts written past the stop left
    no trace in the positions before it). The prompt ends with 40 tokens of the model's
    own greedy stream, which has fallen into a cycle by then, so the drafter has
    matches from the first step on."""
    import shutil
    from conftest import gguf_kv_u32_offset
    path = synth_cached("eng-512", SMALL, 21)
    V = SMALL["n_vocab"]
    base = minfer.prompt_ids(31, 12, V) * 6
    ref = minfer.Engine(path, max_ctx=200)
    ref.prefill(base)
    stream, _ = ref.generate(96)
    ref.close()
    prompt, want, n_gen = base + stream[:40], stream[40:], 56
    # the eos: the continuation's token whose first occurrence in it is the latest
    first = max(want.index(t) for t in set(want))
    assert first >= 3
    stop_path = str(tmp_path / "eos-stop.gguf")
    shutil.copy(path, stop_path)
    with open(stop_path, "r+b") as f:
        f.seek(gguf_kv_u32_offset(stop_path, "tokenizer.ggml.eos_token_id"))
        f.write(np.uint32(want[first]).tobytes())
    res = {}
    for mode, opts in (("plain", dict(spec=0)), ("host", dict(spec=1, persistent=1)),
                       ("host_persistent", dict(spec=1, persistent=2)), ("device", dict(spec=2, persistent=2))):
        say("eos stop at output %d: %s" % (first, mode))
        eng = minfer.Engine(stop_path, max_ctx=200, stop_eos=1, **opts)
        eng.prefill(prompt)
        toks, margins = eng.generate(n_gen)
        st = eng.stats()
        _, _, lg = eng.step(want[first], len(prompt) + first, want_logits=True)
        res[mode] = (toks, margins, lg, st)
        eng.close()
        say("  %d tokens, %d steps, %d drafted, %d accepted" % (len(toks), st["steps"], st["drafted"], st["accepted"]))
    assert res["plain"][0] == want[:first + 1]
    for mode in ("host", "host_persistent", "device"):
        assert res[mode][0] == res["plain"][0], mode
        assert np.array_equal(bits(res[mode][1]), bits(res["plain"][1])), mode
        assert np.array_equal(bits(res[mode][2]), bits(res["plain"][2])), mode
    assert res["device"][3]["accepted"] > 0
    for key in ("steps", "drafted", "accepted"):
        assert res["device"][3][key] == res["host"][3][key], key
