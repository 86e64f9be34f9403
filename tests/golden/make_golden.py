"""Write the golden token streams of the reference cpu_infer (test fixtures).

Runs in the authoring container only: it needs /root/reference (the reference
cpu_infer is compiled from its own sources by `make -C oracle ref`) and writes
small JSON fixtures here. The GGUF inputs are regenerated bit-identically from
their seeds by mi_synth_gguf; the fixture records the file's xxh64 so a test can
prove the regeneration.

    python tests/golden/make_golden.py [config0] [config2] [tiny] [mixed]

`mixed` is the tiny shape with the tensor types of a real Qwen2.5 q4_0 file
(q6_K output.weight, q4_1 ffn_down) and a q8_0 token embedding. `attn` (head_dim
128) and `attn64` (head_dim 64) are attention-sensitive models: q/k biases
N(0, 2) and norm weights 1 + N(0, 0.02) give attention scores of order 1 that
depend on the relative position, so the streams pin RoPE and the GQA head
mapping (with the BASELINE distributions attention is near uniform and a
RoPE sign flip leaves the greedy stream unchanged).
"""
import json
import os
import subprocess
import sys
import time

import xxhash

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "nano-inference_amd"))
import minfer  # noqa: E402

REF = os.path.join(ROOT, "oracle", "_ref", "cpu_infer")
TMP = os.environ.get("MI_TMP", "/tmp/mi")
TINY = dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=4096)
MIXED = dict(head_type=minfer.GT_Q6_K, down_type=minfer.GT_Q4_1, emb_type=minfer.GT_Q8_0)
ATTN = dict(n_layer=2, n_embd=512, n_ff=1024, n_head=4, n_head_kv=2, n_vocab=4096)
SHARP = dict(qk_bias_std=2.0, norm_offset=1.0)


def file_hash(path):
    h = xxhash.xxh64()
    with open(path, "rb") as f:
        while True:
            b = f.read(1 << 24)
            if not b:
                break
            h.update(b)
    return h.hexdigest()


def run(name, shape, mseed, pseed, n_prompt, n_gen, types=None):
    os.makedirs(TMP, exist_ok=True)
    path = os.path.join(TMP, "%s.gguf" % name)
    minfer.synth_gguf(path, shape, mseed, **(types or {}))
    V = (minfer.SHAPES[shape] if isinstance(shape, str) else shape)["n_vocab"]
    ids = minfer.prompt_ids(pseed, n_prompt, V)
    t = time.time()
    r = subprocess.run([REF, path, str(n_gen)] + [str(i) for i in ids], capture_output=True, text=True, check=True)
    toks = [int(x) for x in r.stdout.split()]
    fx = dict(config=name, shape=shape, types=types or {}, model_seed=mseed, prompt_seed=pseed, prompt=ids, n_gen=n_gen,
              tokens=toks, gguf_xxh64=file_hash(path), gguf_bytes=os.path.getsize(path),
              source="reference src/cpu_infer.cpp built by oracle/Makefile (g++ -std=gnu++17 -O3 -march=native -fopenmp)",
              ref_seconds=round(time.time() - t, 1))
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpu_infer_%s.json" % name)
    with open(out, "w") as f:
        json.dump(fx, f, indent=1)
    print(name, "->", out, fx["ref_seconds"], "s")


if __name__ == "__main__":
    which = sys.argv[1:] or ["tiny", "config0", "config2"]
    for w in which:
        if w == "tiny":
            run("tiny", TINY, 7, 8, 8, 64)
        elif w == "mixed":
            run("mixed", TINY, 17, 18, 12, 64, types=MIXED)
        elif w == "attn":
            run("attn", ATTN, 31, 32, 12, 64, types=SHARP)
        elif w == "attn64":
            run("attn64", TINY, 33, 34, 12, 64, types=SHARP)
        else:
            shape, ms, ps, npr, ng = minfer.CONFIGS[w]
            run(w, shape, ms, ps, npr, ng)
