"""Headline benchmark: batch-1 greedy decode tok/s, Qwen2.5-1.5B-shape q4_0, tg128.

    python bench.py [--gpus 1] [--steps 5] [--warmup 1]

Workload: random-init S15 GGUF (hidden 1536, 28 layers,
12/2 heads, hd 128, FFN 8960, vocab 151936) written from a fixed seed, a 64-token
seeded random prompt, then greedy tg128. ONE STEP IS ONE WHOLE tg128: the prompt is
prefilled (untimed, every weight resident in HBM), then 128 decode tokens are timed
(positions 64..191). `--steps K` runs K such generations from the same prompt and
`value` = 128*K / (their summed time); `ms_per_step` = the time of one tg128.
`--warmup W` runs W untimed generations first.

Prints ONE JSON line on stdout. Besides the contract keys it carries:
  roofline      the dominant kernel: the persistent step kernel k_step, one
                launch per token. achieved = algorithmic bytes of one token at
                the mean timed position / the mean launch time, from HIP events
                recorded on the engine's stream around the timed steps; peak =
                MI355X's 8 TB/s HBM. traffic = HBM bytes per launch measured with
                the rocprofv3 FETCH_SIZE and WRITE_SIZE counters (each scaled by
                what it reads for a plain copy of known size), read from the
                committed summary profiles/k_step_config2.md.
                With --persistent 0 the dominant kernel is the gate/up phase.
  step_roofline bytes/token x tok/s against the measured stream-read bandwidth
  stream_gbps   one-launch stream read of a 4 GiB buffer (> the 256 MB MALL)
  phases        the in-kernel profile of one step (device clock stamps per workgroup
                and phase, mi_profile_step): per GEMV phase, weight bytes / the
                phase's time from the previous grid barrier's exit to its own exit,
                against stream_gbps
  gemv          config 1 microbench: each S15 GEMV shape, rotated over copies
                totalling > 512 MB so every launch reads from HBM; sized_stream_us:
                the stream kernel reading the same bytes, launched the same way
  attention_depth  config 3: S15 decode attention at L = 512..32768, 28 rotated
                layer caches, GB/s of K/V read per layer
  speculative   config 2 by speculative decoding (n-gram drafts, T <= 8 verify steps)
  verify_step   config 4: an S3 T = 8 verify step against a T = 1 step at context 1024,
                and the drafter on S3 with a repetitive 1000-token prompt
  cpu_baseline  the oracle's fp32 mode (a restatement of cpu_infer.cpp whose
                token streams equal the reference binary's) on this host's cores

Single measurements for kernel traces: --gemv-only, --attention-only L[,L...] [--mfma],
--verify-only, --copy-calib MIB (counter calibration).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nano-inference_amd"))
import minfer  # noqa: E402

HBM_PEAK_GBPS = 8000.0


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def bytes_per_token(info, pos):
    """Algorithmic HBM bytes of one decode token at position pos: every weight
    once, the residual stream in/out and the QKV vector per layer, the final norm
    input, the fp16 K/V rows of positions 0..pos read plus the new row written."""
    E, L, FF = info.n_embd, info.n_layer, info.n_ff
    kvd = info.n_head_kv * info.head_dim
    qkv = info.n_head * info.head_dim + 2 * kvd
    kv_row = L * 2 * kvd * 2                      # fp16 K and V of one position, all layers
    return (info.weight_bytes + L * 2 * E * 4 + E * 4 + L * qkv * 4 + E * 4
            + kv_row * (pos + 1) + kv_row)


def gemv_microbench(torch, reps=40):
    """config 1: the five S15 GEMV shapes, weights rotated over > 512 MB of copies
    (each rep reads a copy the previous reps did not touch, so the 256 MB MALL holds
    none of it); time per GEMV = graph replay of `reps` launches / reps."""
    import numpy as np
    out = []
    rng = np.random.default_rng(0)
    # ks per shape: the fastest split of K up to 12 (the most split-K partials the engine's
    # residual add takes; down's is the engine's own plan), from a sweep on the box
    shapes = [("qkv", 2048, 1536, 6), ("o", 1536, 1536, 6), ("gate_up", 17920, 1536, 6),
              ("down", 1536, 8960, 10), ("lm_head", 151936, 1536, 2)]
    for name, rows, n_in, ks in shapes:
        nb, cb = n_in // 32, 8
        nbytes = minfer.packed_bytes(rows, nb, cb)
        copies = max(2, -(-(640 << 20) // nbytes))
        w = torch.randint(0, 256, (copies, nbytes), dtype=torch.uint8, device="cuda")
        x = torch.randn(n_in, device="cuda")
        xq = torch.empty(n_in, dtype=torch.int8, device="cuda")
        xd = torch.empty(nb, device="cuda")
        xs8 = torch.empty(nb, dtype=torch.int32, device="cuda")
        minfer.quant_q8(x, xq, xd, xs8)
        part = torch.empty(ks * rows, device="cuda")
        ref = torch.empty(ks * rows, device="cuda")
        for i in range(4):
            minfer.gemv_q4(w[i % copies], rows, nb, cb, ks, xq, xd, xs8, part)
        # the reps launched back to back from a captured graph (ctypes launches from
        # Python would leave the GPU idle between the short kernels); each rep reads
        # another copy of the weights
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(reps):
                minfer.gemv_q4(w[i % copies], rows, nb, cb, ks, xq, xd, xs8, part)
        minfer.gemv_q4(w[(reps - 1) % copies], rows, nb, cb, ks, xq, xd, xs8, ref)
        g.replay()
        torch.cuda.synchronize()
        # bit patterns: the random weight bytes include NaN fp16 scales
        assert torch.equal(part.view(torch.int32), ref.view(torch.int32)), "graph replay differs from the eager launch"
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1000 / reps
        del g
        # a plain read of the same weight bytes, launched the same way (graph replay over the
        # same rotated copies): the stream roofline at this launch's size, fixed costs
        # (launch, first round trip, drain) included, which a 4 GiB stream amortises away
        sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
        gs = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gs):
            for i in range(reps):
                minfer.stream_read(w[i % copies], nbytes, sink)
        gs.replay()
        torch.cuda.synchronize()
        e0.record()
        gs.replay()
        e1.record()
        torch.cuda.synchronize()
        us_s = e0.elapsed_time(e1) * 1000 / reps
        del gs
        alg = rows * nb * 18 + n_in + nb * 4 + rows * 4
        out.append(dict(shape=name, rows=rows, k=n_in, ks=ks, us=round(us, 2), gbps=round(alg / us / 1e3, 1),
                        sized_stream_us=round(us_s, 2), sized_stream_gbps=round(nbytes / us_s / 1e3, 1),
                        frac_of_sized_stream=round(us_s / us, 4)))
        del w
    torch.cuda.empty_cache()
    _ = rng
    return out


def gemv_kernel_us(prefix="kernel_us_"):
    """config-1 kernel durations per shape from the committed rocprofv3 kernel-trace summary
    (prefix "stream_kernel_us_": the plain read of the same bytes)"""
    out = {}
    try:
        with open(os.path.join(ROOT, "profiles", "k_gemv_config1.md")) as f:
            for line in f:
                if line.startswith(prefix):
                    k, v = line[len(prefix):].split(":")
                    out[k.strip()] = float(v)
    except OSError:
        pass
    return out


def traffic_bytes():
    """HBM bytes per k_step launch from the committed rocprofv3 counter summary"""
    try:
        with open(os.path.join(ROOT, "profiles", "k_step_config2.md")) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def stream_bw(torch, gib=4, reps=5):
    buf = torch.empty(gib << 30, dtype=torch.uint8, device="cuda")
    buf.zero_()
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    minfer.stream_read(buf, buf.numel(), sink)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        minfer.stream_read(buf, buf.numel(), sink)
    e1.record()
    torch.cuda.synchronize()
    gbps = buf.numel() * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del buf
    torch.cuda.empty_cache()
    return gbps


def ensure_gguf(name):
    shape, mseed, _, _, _ = minfer.CONFIGS[name]
    tmp = os.path.join(os.environ.get("TMPDIR", "/tmp"), "mi-bench")
    os.makedirs(tmp, exist_ok=True)
    path = os.path.join(tmp, "%s-%d.gguf" % (name, mseed))
    if not os.path.exists(path + ".ok"):
        t = time.time()
        minfer.synth_gguf(path, shape, mseed)
        open(path + ".ok", "w").close()
        log("wrote %s in %.1f s" % (path, time.time() - t))
    return path


def spec_decode(path, prompt, n_gen=128):
    """config2 with speculative decoding (n-gram drafts, verify steps): lossless, so
    the tokens equal the plain run's; wall-clock tok/s of the generation"""
    eng = minfer.Engine(path, max_ctx=len(prompt) + n_gen + 16, spec=1)
    eng.prefill(prompt)
    eng.generate(8)
    eng.prefill(prompt)
    t0 = time.perf_counter()
    toks, _ = eng.generate(n_gen)
    dt = time.perf_counter() - t0
    st = eng.stats()
    eng.close()
    return toks, dict(tok_s=round(n_gen / dt, 2), verify_steps=st["steps"], drafted=st["drafted"],
                      accepted=st["accepted"], tokens_per_step=round(n_gen / max(st["steps"], 1), 3))


def verify_cost(reps=10, modes=(2, 1)):
    """config4: S3 (hidden 2048, 36 layers), context 1024; a T=8 verify step (the
    current token + 7 drafts, TMAX = 8) against a T=1 step at the same position.
    Wall time per mi_step call (upload, step, copy-back), mean of reps. The engine's
    default runs the T=8 step as one persistent launch; t8_per_phase_ms is the same step
    as one launch per phase (persistent=1, same bits)."""
    shape, _, pseed, ctx, _ = minfer.CONFIGS["config4"]
    path = ensure_gguf("config4")
    V = minfer.SHAPES[shape]["n_vocab"]
    prompt = minfer.prompt_ids(pseed, ctx, V)
    toks = minfer.prompt_ids(pseed + 1, 8, V)
    out = {}
    for mode in modes:
        eng = minfer.Engine(path, max_ctx=ctx + 16, persistent=mode)
        eng.prefill(prompt)
        for T in ((1, 8) if mode == 2 else (8,)):
            arg = toks[:T] if T > 1 else toks[0]
            for _ in range(3):
                eng.step(arg, ctx)
            t0 = time.perf_counter()
            for _ in range(reps):
                eng.step(arg, ctx)
            out[(mode, T)] = (time.perf_counter() - t0) / reps * 1e3
        eng.close()
    return dict(workload="config4: S3 q4_0, context 1024, verify T=8 vs T=1", t1_ms=round(out[(2, 1)], 3),
                t8_ms=round(out[(2, 8)], 3), ratio=round(out[(2, 8)] / out[(2, 1)], 3),
                t8_per_phase_ms=round(out[(1, 8)], 3) if (1, 8) in out else None,
                note="T=8 = current token + 7 drafts (TMAX 8, mega.cu:50); the config's 8 drafts + 1 would be T=9")


def verify_spec(n_gen=64):
    """config4's drafter on its own shape: S3, a synthetic repetitive token stream of
    1,000 tokens (a seeded 40-token pattern, 25 times) as the prompt, n_gen tokens by
    speculative decoding (n-gram drafts verified by T <= 8 steps) driven by the host and
    on the device, each checked token for token and margin for margin against plain
    greedy decode. Reports verify steps, drafts, acceptances and tokens per step."""
    shape, _, pseed, _, _ = minfer.CONFIGS["config4"]
    path = ensure_gguf("config4")
    V = minfer.SHAPES[shape]["n_vocab"]
    import numpy as np
    prompt = minfer.prompt_ids(pseed, 40, V) * 25
    out = dict(workload="config4 drafter: S3, 1000-token repetitive prompt (40-token pattern x 25), %d generated" % n_gen)
    ref = None
    for mode, opts in (("plain", dict(spec=0)), ("host", dict(spec=1, persistent=1)),
                       ("host_persistent", dict(spec=1, persistent=2)), ("device", dict(spec=2, persistent=2))):
        eng = minfer.Engine(path, max_ctx=len(prompt) + n_gen + 16, **opts)
        eng.prefill(prompt)
        toks, mg = eng.generate(n_gen)
        st = eng.stats()
        eng.close()
        got = (toks, np.float32(mg).view(np.uint32).tolist())
        if ref is None:
            ref = got
            out["plain_ms"] = round(st["decode_ms"], 3)
            continue
        assert got == ref, "speculative output differs from plain greedy decode (%s)" % mode
        out[mode] = dict(ms=round(st["decode_ms"], 3), verify_steps=st["steps"], drafted=st["drafted"],
                         accepted=st["accepted"], tokens_per_step=round(n_gen / max(st["steps"], 1), 3))
    out["identical_to_plain"] = True
    return out


def attention_depth(torch, lengths=(512, 4096, 16384, 32768), layers=28, reps=3, graph=True, mfma=False):
    """config3: S15 split-KV decode attention (12/2 heads, hd 128), one query, fp16 K/V
    N(0,1) at context L, rotated over 28 layers' caches (28 x 32 MB at L = 32768 > the
    256 MB MALL), the 28 launches replayed from a graph. Algorithmic bytes per layer:
    1024*L (K and V) + q/out. mfma: the matrix-core chunk records (mi_attn_decode_mfma)
    instead of the canonical ones; its result is checked against the canonical one."""
    nh, nkv, hd = 12, 2, 128
    attn = minfer.attn_decode_mfma if mfma else minfer.attn_decode
    res = []
    for L in lengths:
        kc = torch.randn(layers, nkv, L, hd, device="cuda").half()
        vc = torch.randn(layers, nkv, L, hd, device="cuda").half()
        q = torch.randn(nh, hd, device="cuda")
        scratch = torch.zeros(minfer.attn_scratch_floats(nh, hd, L), device="cuda")
        out = torch.empty(nh * hd, device="cuda")
        scale = 1.0 / hd ** 0.5
        for l in range(2):
            attn(q, kc[l], vc[l], nh, nkv, hd, L, L, scale, scratch, out)
        if mfma:
            canon = torch.empty_like(out)
            minfer.attn_decode(q, kc[1], vc[1], nh, nkv, hd, L, L, scale, scratch, canon)
            torch.cuda.synchronize()
            rel = float((out - canon).abs().max() / canon.abs().max())
            assert rel <= 1e-5, "mfma attention off the canonical result by %g" % rel
        # the layers' launches replayed from a captured graph (ctypes launches from
        # Python would leave the GPU idle between the short kernels); the kernel's
        # counters return to zero by themselves, so replays need no reset. graph=False
        # (for kernel traces, which time each launch themselves): eager launches.
        def layer_loop():
            for l in range(layers):
                attn(q, kc[l], vc[l], nh, nkv, hd, L, L, scale, scratch, out)
        g = None
        if graph:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                layer_loop()
            ref = torch.empty_like(out)
            attn(q, kc[layers - 1], vc[layers - 1], nh, nkv, hd, L, L, scale, scratch, ref)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), "graph replay differs from the eager launch"
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            if g is not None:
                g.replay()
            else:
                layer_loop()
        e1.record()
        torch.cuda.synchronize()
        del g
        us = e0.elapsed_time(e1) * 1e3 / (reps * layers)
        byt = 1024 * L + 2 * nh * hd * 4
        res.append(dict(L=L, us_per_layer=round(us, 2), gbps=round(byt / us / 1e3, 1)))
        del kc, vc
    torch.cuda.empty_cache()
    return res


def cpu_model():
    """the host CPU's model name (lscpu's "Model name", from /proc/cpuinfo)"""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(path, prompt, n_prompt=64, n_gen=129):
    """oracle fp32 (cpu_infer semantics) on the host cores: the whole config2
    workload (64-token prompt, 128 decode steps), about 15 s on 16 threads"""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    m = O.Model(path, O.MODE_FP32, max_seq=n_prompt + n_gen + 1, threads=threads)
    _, _, tp, td = m.generate(prompt[:n_prompt], n_gen)
    m.close()
    return dict(value=round((n_gen - 1) / td, 3), unit="tok/s", cores=threads, kind="port", cpu=cpu_model(),
                sample="S15 greedy decode: %d-token prompt (%.1f s) then %d tokens (%d decode steps in %.1f s), "
                       "oracle fp32 = cpu_infer.cpp semantics, OpenMP %d threads on %s" % (
                           n_prompt, tp, n_gen, n_gen - 1, td, threads, cpu_model()))


# q4_0 weight bytes of one layer's GEMV of each phase kind (rows x blocks x 18)
def phase_weight_bytes(info):
    E, FF = info.n_embd, info.n_ff
    qkv = info.n_head * info.head_dim + 2 * info.n_head_kv * info.head_dim
    nbE, nbF = E // 32, FF // 32
    return {"qkv": qkv * nbE * 18, "o": E * nbE * 18, "gate_up": 2 * FF * nbE * 18, "down": E * nbF * 18,
            "lm_head": info.n_vocab * nbE * 18}


def phase_profile(eng, stream_gbps):
    """In-kernel phase times of one persistent step (mi_profile_step: device clock stamps
    of every workgroup). A phase runs from the previous grid barrier's exit to its own
    barrier's exit (the earliest exit over workgroups = when the barrier completed); per
    GEMV kind, the weight bytes of all layers / the summed phase times, against the
    measured stream bandwidth."""
    t = eng.profile_step()
    L = eng.info.n_layer
    exits = [0.0]
    kinds = []
    for l in range(L):
        for k, name in enumerate(("qkv", "attn", "o", "gate_up", "down")):
            exits.append(float(t[:, eng.prof_slot(l, k, 4)].min()))
            kinds.append(name)
    exits.append(float(t[:, eng.prof_slot(L, 0, 4)].min()))
    kinds.append("lm_head")
    wb = phase_weight_bytes(eng.info)
    tot = {}
    for i, name in enumerate(kinds):
        tot[name] = tot.get(name, 0.0) + exits[i + 1] - exits[i]
    out = []
    for name in ("qkv", "attn", "o", "gate_up", "down", "lm_head"):
        us = tot[name]
        n = 1 if name == "lm_head" else L
        d = dict(phase=name, us_per_layer=round(us / n, 2), us_total=round(us, 1))
        if name in wb:
            gbps = wb[name] * n / (us * 1e-6) / 1e9
            d.update(weight_bytes=wb[name], gbps=round(gbps, 1), frac_of_stream=round(gbps / stream_gbps, 4))
        out.append(d)
    return out, round(exits[-1], 1)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5, help="timed tg128 generations")
    ap.add_argument("--warmup", type=int, default=1, help="untimed tg128 generations before them")
    ap.add_argument("--tg", type=int, default=128, help="decode tokens per step (the metric is tg128)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-micro", action="store_true")
    ap.add_argument("--persistent", type=int, default=1)
    ap.add_argument("--no-extra", action="store_true", help="skip the speculative and verify-step measurements")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB three times (calibrates the "
                         "rocprofv3 FETCH_SIZE/WRITE_SIZE counters) and exit")
    ap.add_argument("--attention-only", type=str, default="", metavar="L[,L...]",
                    help="only run the config3 attention-at-depth measurement at these context "
                         "lengths, print its JSON and exit")
    ap.add_argument("--mfma", action="store_true",
                    help="with --attention-only: the matrix-core chunk records (mi_attn_decode_mfma)")
    ap.add_argument("--eager", action="store_true",
                    help="with --attention-only: launch eagerly instead of replaying a graph (for kernel traces)")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only run the config1 GEMV microbench, print its JSON and exit (for kernel traces)")
    ap.add_argument("--verify-only", action="store_true",
                    help="only run the config4 verify-step cost (T=8 vs T=1), print its JSON and exit "
                         "(for kernel traces)")
    ap.add_argument("--verify-persistent-only", action="store_true",
                    help="with --verify-only: skip the per-phase launches (for counter runs)")
    args = ap.parse_args()
    if args.verify_only:
        res = verify_cost(modes=(2,) if args.verify_persistent_only else (2, 1))
        log("verify step: %s" % res)
        print(json.dumps({"verify_step": res}), flush=True)
        return
    if args.gemv_only:
        import torch
        res = gemv_microbench(torch)
        for m in res:
            log("gemv %-8s %6d x %5d: %8.2f us  %7.1f GB/s  (a read of the same bytes: %.2f us)" % (
                m["shape"], m["rows"], m["k"], m["us"], m["gbps"], m["sized_stream_us"]))
        print(json.dumps({"gemv": res}), flush=True)
        return
    if args.attention_only:
        import torch
        lens = tuple(int(x) for x in args.attention_only.split(","))
        res = attention_depth(torch, lengths=lens, graph=not args.eager, mfma=args.mfma)
        for a in res:
            log("attention L=%-6d %8.2f us/layer  %7.1f GB/s" % (a["L"], a["us_per_layer"], a["gbps"]))
        print(json.dumps({"attention_depth": res}), flush=True)
        return
    if args.copy_calib:
        import torch
        src = torch.ones(args.copy_calib << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes": src.numel(), "reps": 3}), flush=True)
        return
    if args.gpus != 1:
        print("bench.py: batch-1 decode runs on one GPU; --gpus %d is not supported here "
              "(no collective or second-GPU path is built)" % args.gpus, file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    shape, mseed, pseed, n_prompt, _ = minfer.CONFIGS["config2"]
    path = ensure_gguf("config2")
    V = minfer.SHAPES[shape]["n_vocab"]
    prompt = minfer.prompt_ids(pseed, n_prompt, V)
    tg = args.tg
    t = time.time()
    eng = minfer.Engine(path, max_ctx=n_prompt + tg + 16, persistent=args.persistent)
    info = eng.info
    log("loaded in %.1f s: plan cb=%s ks=%s, %d CUs, weights %d B" % (time.time() - t, list(info.plan_cb),
                                                                     list(info.plan_ks), info.n_cu, info.weight_bytes))

    def one_tg():
        """prefill the prompt (untimed), then one timed tg: 1 + tg tokens, the first
        being the prefill's prediction, so exactly tg decode steps (positions 64..)"""
        eng.prefill(prompt)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        toks, margins = eng.generate(tg + 1)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        st = eng.stats()
        assert st["steps"] == tg
        return toks, dt, st["decode_ms"]

    for _ in range(args.warmup):
        one_tg()
    wall = dev_ms = 0.0
    toks = None
    for k in range(args.steps):
        tk, dt, dms = one_tg()
        if toks is None:
            toks = tk
        assert tk == toks, "tg%d stream differs between steps" % tg
        wall += dt
        dev_ms += dms
        log("step %d: tg%d in %.2f ms wall (%.2f ms device)" % (k, tg, dt * 1e3, dms))
    ntok = tg * args.steps
    ms_per_step = wall * 1e3 / args.steps
    tok_s = ntok / wall
    log("decode: %d x tg%d = %d tokens in %.2f ms wall (%.2f ms device) = %.1f tok/s" % (
        args.steps, tg, ntok, wall * 1e3, dev_ms, tok_s))
    mean_pos = n_prompt + (tg - 1) / 2.0
    bpt = bytes_per_token(info, mean_pos)
    if info.persistent:
        # dominant kernel: k_step, one launch per token; its mean duration comes
        # from the engine's HIP events around the timed launches on its stream
        k_us = dev_ms * 1e3 / ntok
        k_bytes = int(bpt)
        kname = "k_step (persistent decode step, 1 launch/token, %d workgroups)" % info.n_cu
    else:
        E, FF = info.n_embd, info.n_ff
        k_us = eng.time_phase("gate_up", layer=info.n_layer // 2, reps=50) * 1e3
        k_bytes = 2 * FF * (E // 32) * 18 + E * 4 * (2 + info.plan_ks[1]) + info.plan_ks[2] * 2 * FF * 4
        kname = "k_gu (gate/up GEMV phase, %d launches/token)" % info.n_layer
    k_gbps = k_bytes / (k_us * 1e-6) / 1e9
    log("%s: %.2f us per launch, %.1f GB/s" % (kname, k_us, k_gbps))
    stream = stream_bw(torch)
    log("stream read: %.1f GB/s" % stream)
    phases, prof_total = (None, None)
    if info.persistent:
        phases, prof_total = phase_profile(eng, stream)
        for ph in phases:
            log("phase %-8s %7.2f us/layer%s" % (ph["phase"], ph["us_per_layer"],
                                                 "  %7.1f GB/s = %.1f%% of stream" % (ph["gbps"], 100 * ph["frac_of_stream"])
                                                 if "gbps" in ph else ""))
    eng.close()
    del eng
    micro = [] if args.no_micro else gemv_microbench(torch)
    ktr, kst = gemv_kernel_us(), gemv_kernel_us("stream_kernel_us_")
    for m in micro:
        m["frac_of_stream"] = round(m["gbps"] / stream, 4)
        if m["shape"] in ktr:          # kernel duration alone (rocprofv3 trace, profiles/k_gemv_config1.md)
            alg = m["gbps"] * m["us"] * 1e3
            m["kernel_us"] = ktr[m["shape"]]
            m["kernel_gbps"] = round(alg / ktr[m["shape"]] / 1e3, 1)
            m["kernel_frac_of_stream"] = round(m["kernel_gbps"] / stream, 4)
            if m["shape"] in kst:      # against a read of the same bytes, both from the same trace
                m["sized_stream_kernel_us"] = kst[m["shape"]]
                m["kernel_frac_of_sized_stream"] = round(kst[m["shape"]] / ktr[m["shape"]], 4)
        log("gemv %-8s %6d x %5d: %8.2f us  %7.1f GB/s  (a read of the same bytes: %.2f us)" % (
            m["shape"], m["rows"], m["k"], m["us"], m["gbps"], m["sized_stream_us"]))
    attn = [] if args.no_micro else attention_depth(torch)
    for a in attn:
        log("attention L=%-6d %8.2f us/layer  %7.1f GB/s" % (a["L"], a["us_per_layer"], a["gbps"]))
    attn_mx = [] if args.no_micro else attention_depth(torch, mfma=True)
    for a in attn_mx:
        log("attention (mfma records) L=%-6d %8.2f us/layer  %7.1f GB/s" % (a["L"], a["us_per_layer"], a["gbps"]))
    for a in attn + attn_mx:          # against the stream roofline measured in this run
        a["frac_of_stream"] = round(a["gbps"] / stream, 4)
    spec = verify = None
    if not args.no_extra:
        stoks, spec = spec_decode(path, prompt, tg + 1)
        spec["identical_to_plain"] = stoks == toks
        log("speculative decode: %s" % spec)
        verify = verify_cost()
        verify["drafter"] = verify_spec()
        log("verify step: %s" % verify)
    cpu = None if args.no_cpu else cpu_baseline(path, prompt)
    if cpu:
        log("cpu baseline: %s" % cpu)
    achieved_step = bpt * tok_s / 1e9
    rec = {
        "metric": "batch-1 decode tok/s, Qwen2.5-1.5B q4_0 tg%d; GEMV HBM GB/s vs peak" % tg,
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_0 weights x int8 activations, int32 dot, fp32 accumulate/softmax, fp16 KV",
        "data": "synthetic: seeded random-init GGUF (mi_synth_gguf seed %d), seeded random prompt" % mseed,
        "config": {"workload": "config2: Qwen2.5-1.5B-architecture q4_0 batch-1 greedy decode, 64-token prompt, "
                               "tg%d; one step = one whole tg%d (%d decode tokens timed), %d steps" % (tg, tg, tg,
                                                                                                     args.steps),
                   "shape": "S15 E1536 L28 H12/2 hd128 FF8960 V151936", "global_batch": 1,
                   "prompt": n_prompt, "tokens_per_step": tg,
                   "step_mode": "persistent" if info.persistent else "one launch per phase",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": kname,
                     "achieved": round(k_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(k_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": traffic_bytes() if info.persistent else None,
                     "bytes_per_launch": k_bytes, "us_per_launch": round(k_us, 3)},
        "step_roofline": {"bytes_per_token": int(bpt), "achieved_gbps": round(achieved_step, 1),
                          "stream_gbps": round(stream, 1), "frac_of_stream": round(achieved_step / stream, 4),
                          "roofline_tok_s": round(stream * 1e9 / bpt, 1)},
        "stream_gbps": round(stream, 1),
        "phases": phases, "profiled_step_us": prof_total,
        "gemv": micro,
        "attention_depth": attn,
        "attention_depth_mfma": attn_mx,
        "device_decode_ms": round(dev_ms, 3),
        "cpu_baseline": cpu,
        "speculative": spec,
        "verify_step": verify,
        "tokens_head": toks[:8],
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
