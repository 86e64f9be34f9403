"""The CPU oracle behind the engine's C ABI (oracle/mi_abi.c, loaded through
tests/engine_abi.py exactly as the HIP library is): in fp32 mode mi_prefill +
mi_generate reproduce the reference cpu_infer's committed token streams, mi_teacher's
predictions past the prompt are those streams, and the entry points return the
status codes include/minfer.h documents. The GPU tests run the same call sequence on
both backends (tests/test_gpu_backend_swap.py)."""
import json
import os

import numpy as np
import pytest

import engine_abi as A
import minfer
from conftest import synth_cached

HERE = os.path.dirname(os.path.abspath(__file__))


def fixture(name):
    with open(os.path.join(HERE, "golden", "cpu_infer_%s.json" % name)) as f:
        fx = json.load(f)
    return fx, synth_cached(fx["config"], fx["shape"], fx["model_seed"], **fx.get("types", {}))


@pytest.fixture(scope="module", autouse=True)
def fp32_mode():
    A.oracle_mode(0)
    yield
    A.oracle_mode(1)


@pytest.mark.parametrize("name", ["tiny", "attn64", "mixed"])
def test_oracle_abi_reproduces_reference_streams(name):
    fx, path = fixture(name)
    eng = A.AbiEngine(A.ORACLE_LIB, path, max_ctx=len(fx["prompt"]) + fx["n_gen"] + 8)
    first, _ = eng.prefill(fx["prompt"])
    toks, _ = eng.generate(fx["n_gen"])
    assert first == fx["tokens"][0]
    assert toks.tolist() == fx["tokens"], name
    # teacher forcing over prompt + stream: the prediction after position i is token i+1
    pred, _ = eng.teacher(fx["prompt"] + fx["tokens"])
    n = len(fx["prompt"])
    assert pred[n - 1:-1].tolist() == fx["tokens"]
    eng.close()


def test_oracle_abi_multi_token_step_equals_single_steps():
    fx, path = fixture("tiny")
    eng = A.AbiEngine(A.ORACLE_LIB, path, max_ctx=64)
    eng.prefill(fx["prompt"])
    toks = fx["tokens"][:6]
    pos = len(fx["prompt"])
    am, mg, lg = eng.step(toks, pos, want_logits=True)
    for t in range(len(toks)):
        a, m, l1 = eng.step(toks[t:t + 1], pos + t, want_logits=True)
        assert a[0] == am[t] and np.array_equal(l1[0].view(np.uint32), lg[t].view(np.uint32))
    eng.close()


def test_oracle_abi_status_codes():
    fx, path = fixture("tiny")
    with pytest.raises(minfer.MinferError) as e:
        A.AbiEngine(A.ORACLE_LIB, path + ".missing")
    assert e.value.code == -2                                    # MI_ERR_IO
    with pytest.raises(minfer.MinferError) as e:
        A.AbiEngine(A.ORACLE_LIB, path, tchunk=9)
    assert e.value.code == -1                                    # MI_ERR_ARG
    eng = A.AbiEngine(A.ORACLE_LIB, path, max_ctx=32)
    with pytest.raises(minfer.MinferError) as e:
        eng.generate(4)
    assert e.value.code == -7                                    # MI_ERR_STATE: generate before prefill
    with pytest.raises(minfer.MinferError) as e:
        eng.prefill([fx["shape"]["n_vocab"]])
    assert e.value.code == -1                                    # token out of range
    eng.prefill(fx["prompt"])
    with pytest.raises(minfer.MinferError) as e:
        eng.step([1] * 9, len(fx["prompt"]))
    assert e.value.code == -1                                    # T outside 1..8
    with pytest.raises(minfer.MinferError) as e:
        eng.step([1], len(fx["prompt"]) + 1)
    assert e.value.code == -1                                    # past the current length
    with pytest.raises(minfer.MinferError) as e:
        eng.generate(40)
    assert e.value.code == -1                                    # beyond the capacity
    eng.close()
