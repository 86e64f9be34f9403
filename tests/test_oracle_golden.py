"""Pins the oracle's fp32 mode against the reference cpu_infer's own token streams.

The fixtures (tests/golden/cpu_infer_*.json) were written by
tests/golden/make_golden.py, which compiles src/cpu_infer.cpp from the reference
tree (oracle/Makefile `ref`) and runs it on seeded synthetic GGUFs. Here the same
GGUFs are regenerated (their xxh64 must match, proving the regeneration) and the
oracle's cpu_infer restatement must emit the identical greedy stream. The q8act
mode (the GPU engine's numerics) is then checked against fp32 within the int8
activation error.
"""
import json
import os

import numpy as np
import pytest

import minfer
import oracle_lib as O
from conftest import synth_cached

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with open(os.path.join(GOLDEN, "cpu_infer_%s.json" % name)) as f:
        return json.load(f)


def file_hash(path):
    import xxhash
    h = xxhash.xxh64()
    with open(path, "rb") as f:
        for b in iter(lambda: f.read(1 << 24), b""):
            h.update(b)
    return h.hexdigest()


def model_path(fx):
    return synth_cached(fx["config"], fx["shape"], fx["model_seed"], **fx.get("types", {}))


def check_stream(fx, n=None):
    path = model_path(fx)
    assert file_hash(path) == fx["gguf_xxh64"], "synthetic GGUF regeneration differs"
    V = (minfer.SHAPES[fx["shape"]] if isinstance(fx["shape"], str) else fx["shape"])["n_vocab"]
    assert minfer.prompt_ids(fx["prompt_seed"], len(fx["prompt"]), V) == fx["prompt"]
    n = n or fx["n_gen"]
    m = O.Model(path, O.MODE_FP32, max_seq=len(fx["prompt"]) + n + 1)
    toks, _, _, _ = m.generate(fx["prompt"], n)
    m.close()
    assert toks == fx["tokens"][:n]


def test_tiny_stream_matches_reference_cpu_infer():
    check_stream(load("tiny"))


def test_mixed_types_stream_matches_reference_cpu_infer():
    """q6_K output.weight, q4_1 ffn_down and a q8_0 embedding (gguf.h:85-142): the
    fp32 oracle's dequantization of each type must give the reference's stream"""
    fx = load("mixed")
    assert fx["types"] == {"head_type": 14, "down_type": 3, "emb_type": 8}
    check_stream(fx)


@pytest.mark.slow
def test_config0_stream_matches_reference_cpu_infer():
    check_stream(load("config0"))


@pytest.mark.slow
def test_config2_stream_matches_reference_cpu_infer():
    """all 128 tokens of config 2 (S15, 64-token prompt; ~30 s on 8 cores)"""
    check_stream(load("config2"))


@pytest.mark.parametrize("name", ["attn", "attn64"])
def test_attention_sensitive_stream_matches_reference_cpu_infer(name):
    """Models whose attention matters (q/k biases N(0, 2), norm weights 1 + N(0, 0.02):
    scores of order 1 that depend on the relative position; head_dim 128 and 64, 4 query
    heads on 2 kv heads). The fp32 oracle must give the reference's stream; a RoPE sign
    flip or the head mapping hh % n_kv instead of hh / G (cpu_infer.cpp:49-61, 123)
    leaves it within the first 4 tokens, which the default distributions do not."""
    fx = load(name)
    assert fx["types"] == {"qk_bias_std": 2.0, "norm_offset": 1.0}
    check_stream(fx)


# q8act vs fp32 logits on the attention-sensitive models: the int8 activations leave a
# max-abs error of 1.2-1.5% of the logit range (measured); a flipped RoPE sign or a
# swapped GQA head mapping in either mode moves them by 78-213% (measured on mutated
# copies of the oracle), so 5% separates the two by more than an order of magnitude
Q8ACT_VS_FP32_MAX_REL = 0.05


@pytest.mark.parametrize("name", ["attn", "attn64"])
def test_q8act_logits_close_to_fp32_attention_sensitive(name):
    """the q8act composition (RoPE application, GQA head mapping, merge of attention
    chunks, fp16 KV) against the fp32 mode that the reference's stream pins, at the 60
    positions of the prompt and the reference's continuation"""
    fx = load(name)
    path = model_path(fx)
    seq = fx["prompt"] + fx["tokens"]
    plan = O.Plan.make([8] * 5, [1, 1, 1, 1, 1])
    a = O.Model(path, O.MODE_FP32, max_seq=100)
    b = O.Model(path, O.MODE_Q8ACT, plan=plan, max_seq=100)
    worst = 0.0
    for pos, tok in enumerate(seq[:60]):
        _, _, la = a.forward(tok, pos, True)
        _, _, lb = b.forward(tok, pos, True)
        worst = max(worst, float(np.abs(la - lb).max() / np.abs(la).max()))
        assert np.corrcoef(la, lb)[0, 1] > 0.999, pos
    assert worst < Q8ACT_VS_FP32_MAX_REL, worst


def test_q8act_logits_close_to_fp32():
    fx = load("tiny")
    path = model_path(fx)
    plan = O.Plan.make([4] * 5, [1, 2, 2, 4, 1])
    a = O.Model(path, O.MODE_FP32, max_seq=64)
    b = O.Model(path, O.MODE_Q8ACT, plan=plan, max_seq=64)
    agree = 0
    for pos, tok in enumerate(fx["prompt"]):
        ta, _, la = a.forward(tok, pos, True)
        tb, _, lb = b.forward(tok, pos, True)
        agree += ta == tb
        # int8 activations: per-block rounding noise of a few 1e-3 relative per GEMV
        rel = np.abs(la - lb).max() / np.abs(la).max()
        assert rel < 0.08, rel
        assert np.corrcoef(la, lb)[0, 1] > 0.995
    assert agree >= len(fx["prompt"]) - 2


def test_q8act_plan_changes_only_rounding():
    fx = load("tiny")
    path = model_path(fx)
    p1 = O.Model(path, O.MODE_Q8ACT, plan=O.Plan.make([8] * 5, [1, 1, 1, 1, 1]), max_seq=16)
    p2 = O.Model(path, O.MODE_Q8ACT, plan=O.Plan.make([4] * 5, [2, 2, 2, 4, 2]), max_seq=16)
    _, _, la = p1.forward(fx["prompt"][0], 0, True)
    _, _, lb = p2.forward(fx["prompt"][0], 0, True)
    assert not np.array_equal(la, lb)              # the plan is a real parameter of the order
    assert np.abs(la - lb).max() <= 1e-3 * np.abs(la).max()
