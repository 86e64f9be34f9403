"""The parity harness with the backends swapped (the drop-in boundary's own test): one
call sequence through the engine's C ABI (tests/engine_abi.py `session`: mi_prefill,
mi_generate, a multi-token mi_step with logits at the end of the context, mi_teacher over
the whole sequence) runs on the HIP library and on the CPU oracle's implementation of the
same ABI (oracle/mi_abi.c, q8act mode, given the reduction plan the HIP engine reports).
Every token, margin and logit that comes back is bit-identical, whatever step mode,
prompt chunking or speculation the HIP engine uses (they change no bits)."""
import json
import os

import numpy as np
import pytest

import engine_abi as A
import minfer
from conftest import synth_cached

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
TINY = dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=4096)


@pytest.fixture(scope="module", autouse=True)
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def model(name):
    if name == "tiny":
        return synth_cached("eng-256", TINY, 7), TINY["n_vocab"]
    if name == "config0":
        shape = minfer.SHAPES["S05"]
        return synth_cached("config0", shape, minfer.CONFIGS["config0"][1]), shape["n_vocab"]
    with open(os.path.join(HERE, "golden", "cpu_infer_%s.json" % name)) as f:
        fx = json.load(f)
    return synth_cached(fx["config"], fx["shape"], fx["model_seed"], **fx["types"]), fx["shape"]["n_vocab"]


@pytest.mark.parametrize("name,opts", [("tiny", dict(tchunk=8, persistent=1)),
                                       ("attn", dict(tchunk=5, persistent=2, spec=1)),
                                       ("attn64", dict(tchunk=8, persistent=0)),
                                       ("config0", dict(tchunk=8, persistent=1))])
def test_hip_and_oracle_backends_agree(name, opts):
    path, V = model(name)
    prompt = minfer.prompt_ids(61, 21, V)
    step_toks = minfer.prompt_ids(62, 8, V)
    hip = A.AbiEngine(A.HIP_LIB, path, max_ctx=96, **opts)
    plan = (list(hip.info.plan_cb), list(hip.info.plan_ks))
    A.oracle_mode(1, plan)
    orc = A.AbiEngine(A.ORACLE_LIB, path, max_ctx=96)
    rh = A.session(hip, prompt, 24, step_toks)
    ro = A.session(orc, prompt, 24, step_toks)
    hip.close()
    orc.close()
    assert rh["first"] == ro["first"] and np.float32(rh["m0"]).view(np.uint32) == np.float32(ro["m0"]).view(np.uint32)
    for k in ("toks", "step_argmax", "pred"):
        assert np.array_equal(rh[k], ro[k]), (name, k)
    for k in ("mg", "step_margin", "step_logits", "teacher_margin"):
        assert np.array_equal(np.asarray(rh[k]).view(np.uint32), np.asarray(ro[k]).view(np.uint32)), (name, k)
