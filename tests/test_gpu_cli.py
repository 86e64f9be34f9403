"""GPU checks of the host CLI (the reference's process interface: argv
`<model.gguf> <n_gen> <id...>`, IDs on stdout with RAWIDS=1, text otherwise, stat
lines on stderr; cuda_infer.cu:845-868, 1170-1200) and of chunked prefill (prompt
chunks of tchunk tokens through the multi-token step, cuda_infer.cu:1133-1144), whose
results must equal one step per token bit for bit.
"""
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import minfer
from conftest import synth_cached

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "nano-inference_amd", "_build", "minfer")
TINY = dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=4096)


def say(*a):
    print("[gpu-cli]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def run_cli(path, n_gen, ids, **env):
    e = dict(os.environ)
    e.update({k: str(v) for k, v in env.items()})
    r = subprocess.run([CLI, path, str(n_gen)] + [str(i) for i in ids], capture_output=True, env=e, timeout=120)
    assert r.returncode == 0, r.stderr.decode(errors="replace")
    return r.stdout, r.stderr.decode(errors="replace")


def engine_stream(path, ids, n_gen, **opts):
    eng = minfer.Engine(path, max_ctx=len(ids) + n_gen + 16, **opts)
    eng.prefill(ids)
    toks, _ = eng.generate(n_gen)
    texts = [eng.token_text(t) for t in toks]
    eos = eng.info.eos
    eng.close()
    return toks, texts, eos


def test_cli_raw_ids_match_the_engine():
    path = synth_cached("eng-256", TINY, 7)
    ids = minfer.prompt_ids(3, 20, TINY["n_vocab"])
    say("cli RAWIDS=1, 40 tokens")
    out, err = run_cli(path, 40, ids, RAWIDS=1)
    toks, _, _ = engine_stream(path, ids, 40)
    assert [int(x) for x in out.split()] == toks
    assert out.endswith(b"\n")
    assert re.search(r"prefill: 20 tok in [0-9.]+ ms", err)
    # the rate counts the tokens of the 39 decode steps (the first is the prefill's)
    assert re.search(r"decode: 39 tok in [0-9.]+ ms = [0-9.]+ tok/s", err)


def test_cli_text_mode_streams_token_text():
    path = synth_cached("eng-256", TINY, 7)
    ids = minfer.prompt_ids(4, 12, TINY["n_vocab"])
    say("cli text mode, 30 tokens")
    out, err = run_cli(path, 30, ids)
    toks, texts, eos = engine_stream(path, ids, 30)
    n = toks.index(eos) if eos in toks else len(toks)
    assert out == b"".join(texts[:n]) + b"\n"
    # decode steps: one per emitted token after the prefill's (an eos is emitted, not printed)
    steps = n if eos in toks else n - 1
    assert re.search(r"decode: %d tok in" % steps, err)


def test_cli_spec_and_per_phase_give_the_same_ids():
    path = synth_cached("eng-256", TINY, 7)
    pattern = minfer.prompt_ids(31, 10, TINY["n_vocab"])
    ids = pattern * 4
    say("cli SPEC=1 / PERSISTENT=0 vs plain")
    plain, _ = run_cli(path, 48, ids, RAWIDS=1)
    spec, err = run_cli(path, 48, ids, RAWIDS=1, SPEC=1)
    phases, _ = run_cli(path, 48, ids, RAWIDS=1, PERSISTENT=0)
    assert spec == plain and phases == plain
    m = re.search(r"(\d+) generation steps, ([0-9.]+) tokens/step \| drafted (\d+), accepted (\d+)", err)
    assert m and int(m.group(1)) <= 48 and int(m.group(3)) > 0


@pytest.mark.parametrize("persistent", [1, 0])
def test_chunked_prefill_equals_single_steps(persistent):
    path = synth_cached("eng-256", TINY, 7)
    ids = minfer.prompt_ids(8, 37, TINY["n_vocab"])
    say("chunked prefill, 37-token prompt, persistent=%d" % persistent)
    res = {}
    for tchunk in (1, 3, 8):
        eng = minfer.Engine(path, max_ctx=128, tchunk=tchunk, persistent=persistent)
        first, mg = eng.prefill(ids)
        a, m, lg = eng.step(first, len(ids), want_logits=True)
        toks, mgs = eng.generate(10)
        st = eng.stats()
        eng.close()
        res[tchunk] = (first, int(bits(mg)), a, int(bits(m)), bits(lg).tobytes(), toks, bits(mgs).tobytes())
        say("tchunk %d: prefill %.2f ms" % (tchunk, st["prefill_ms"]))
    assert res[3] == res[1] and res[8] == res[1]


def test_cli_teacher_mode():
    """TEACHER=<k> (mega.cu:28-29, 1192-1205): the summary line with the top-1 agreement
    and the exactness hash, the same hash for every TCHUNK and equal to mi_pred_hash of
    the engine's own teacher-forced predictions; fed the engine's greedy stream, the
    agreement past the prompt is total."""
    path = synth_cached("eng-256", TINY, 7)
    prompt = minfer.prompt_ids(9, 10, TINY["n_vocab"])
    toks, _, _ = engine_stream(path, prompt, 24)
    seq = list(prompt) + toks
    eng = minfer.Engine(path, max_ctx=len(seq) + 16)
    pred, mg = eng.teacher(seq)
    eng.close()
    want = minfer.pred_hash(pred, mg)
    pat = re.compile(r"teacher-forced top-1 agreement: (\d+)/(\d+) \| (\d+) positions in [\d.]+ ms "
                     r"\([\d.]+ ms per (\d+)-token step\) \| logit hash ([0-9a-f]{16})")
    for tchunk in (1, 4, 8):
        say("cli teacher tchunk", tchunk)
        out, err = run_cli(path, 0, seq, TEACHER=len(prompt), TCHUNK=tchunk)
        m = pat.search(err)
        assert m, err
        agree, total, npos, chunk, hsh = int(m.group(1)), int(m.group(2)), int(m.group(3)), int(m.group(4)), m.group(5)
        assert (agree, total, npos, chunk) == (len(seq) - len(prompt), len(seq) - len(prompt), len(seq), tchunk)
        assert int(hsh, 16) == want
        assert out.strip() == b""
