"""Python host binding of the MI355X engine (ctypes over include/minfer.h).

Mirrors the reference engine's interface for the batch-1 token loop: load a GGUF,
prefill a prompt, step tokens, generate greedily (src/cuda_infer.cu:844-1200,
src/mega.cu:1005-1243), with the same argument meaning: int32 token IDs,
positions counted from 0, greedy argmax with the lowest index on ties. Failures
raise MinferError carrying the engine's message instead of exiting. The library
is the in-tree build (nano-inference_amd/_build/libminfer.so); there is no
fallback: if it is missing, importing the engine raises.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB_PATH = os.path.join(PKG, "_build", "libminfer.so")

MI_OK = 0
ERRORS = {-1: "argument", -2: "io", -3: "format", -4: "shape", -5: "device", -6: "oom", -7: "state"}


class MinferError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("minfer %s error (%d): %s" % (ERRORS.get(code, "unknown"), code, msg))
        self.code = code


class Opts(C.Structure):
    _fields_ = [("max_ctx", C.c_int32), ("tchunk", C.c_int32), ("spec", C.c_int32), ("ngmax", C.c_int32),
                ("spec_slope", C.c_float), ("persistent", C.c_int32), ("stop_eos", C.c_int32), ("device", C.c_int32),
                ("graphs", C.c_int32)]


class ModelInfo(C.Structure):
    _fields_ = [("n_layer", C.c_int32), ("n_embd", C.c_int32), ("n_ff", C.c_int32), ("n_head", C.c_int32),
                ("n_head_kv", C.c_int32), ("head_dim", C.c_int32), ("n_vocab", C.c_int32), ("eos", C.c_int32),
                ("rope_base", C.c_float), ("rms_eps", C.c_float), ("max_ctx", C.c_int32),
                ("plan_cb", C.c_int32 * 5), ("plan_ks", C.c_int32 * 5), ("attn_chunk", C.c_int32),
                ("kv_f16", C.c_int32), ("n_cu", C.c_int32), ("persistent", C.c_int32), ("weight_bytes", C.c_uint64),
                ("coop", C.c_int32)]


class Stats(C.Structure):
    _fields_ = [("steps", C.c_int32), ("tokens", C.c_int32), ("decode_ms", C.c_double), ("prefill_ms", C.c_double),
                ("drafted", C.c_int32), ("accepted", C.c_int32)]


class SynthShape(C.Structure):
    _fields_ = [("n_layer", C.c_int32), ("n_embd", C.c_int32), ("n_ff", C.c_int32), ("n_head", C.c_int32),
                ("n_head_kv", C.c_int32), ("n_vocab", C.c_int32), ("rope_base", C.c_float), ("rms_eps", C.c_float),
                ("emb_type", C.c_int32), ("head_type", C.c_int32), ("down_type", C.c_int32), ("tied", C.c_int32),
                ("qk_bias_std", C.c_float), ("norm_offset", C.c_float)]


TOKEN_CB = C.CFUNCTYPE(C.c_int, C.c_int32, C.c_void_p)

# every symbol include/minfer.h declares, with its ctypes signature
_P = C.c_void_p
SIGNATURES = {
    "mi_default_opts": (None, [C.POINTER(Opts)]),
    "mi_load": (C.c_int, [C.c_char_p, C.POINTER(Opts), C.POINTER(_P)]),
    "mi_free": (None, [_P]),
    "mi_last_error": (C.c_char_p, [_P]),
    "mi_info": (C.c_int, [_P, C.POINTER(ModelInfo)]),
    "mi_prefill": (C.c_int, [_P, C.POINTER(C.c_int32), C.c_int32, C.POINTER(C.c_int32), C.POINTER(C.c_float)]),
    "mi_step": (C.c_int, [_P, C.POINTER(C.c_int32), C.c_int32, C.c_int32, C.POINTER(C.c_int32),
                          C.POINTER(C.c_float), C.POINTER(C.c_float)]),
    "mi_generate": (C.c_int, [_P, C.c_int32, C.POINTER(C.c_int32), C.POINTER(C.c_float), C.POINTER(C.c_int32),
                              TOKEN_CB, _P]),
    "mi_get_stats": (C.c_int, [_P, C.POINTER(Stats)]),
    "mi_time_phase": (C.c_int, [_P, C.c_int32, C.c_int32, C.c_int32, C.POINTER(C.c_double)]),
    "mi_profile_step": (C.c_int, [_P, C.POINTER(C.c_double), C.c_int32]),
    "mi_barrier_cost": (C.c_int, [C.c_int32, C.c_int32, C.POINTER(C.c_double)]),
    "mi_debug_flag_barrier": (C.c_int, [_P]),
    "mi_synth_gguf": (C.c_int, [C.c_char_p, C.POINTER(SynthShape), C.c_uint64]),
    "mi_check_layout": (C.c_int, [C.POINTER(SynthShape), C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_char_p,
                                  C.c_int32]),
    "mi_q4_packed_bytes": (C.c_size_t, [C.c_int32, C.c_int32, C.c_int32]),
    "mi_q4_pack": (C.c_int, [_P, C.c_int32, C.c_int32, C.c_int32, _P]),
    "mi_quant_q8": (C.c_int, [_P, C.c_int32, _P, _P, _P, _P]),
    "mi_gemv_q4": (C.c_int, [_P, C.c_int32, C.c_int32, C.c_int32, C.c_int32, _P, _P, _P, _P, _P, _P]),
    "mi_q4_block_isums": (C.c_int, [_P, C.c_int32, C.c_int32, C.c_int32, _P, _P, _P]),
    "mi_attn_decode": (C.c_int, [_P, _P, _P, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_float,
                                 _P, _P, _P]),
    "mi_attn_scratch_floats": (C.c_size_t, [C.c_int32, C.c_int32, C.c_int32]),
    "mi_attn_decode_mfma": (C.c_int, [_P, _P, _P, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_float,
                                 _P, _P, _P]),
    "mi_attn_decode_noalloc": (C.c_int, [_P, _P, _P, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                         C.c_float, _P, _P]),
    "mi_stream_read": (C.c_int, [_P, C.c_size_t, _P, _P]),
    "mi_stream_sync": (C.c_int, [_P]),
    "mi_device_count": (C.c_int, [C.POINTER(C.c_int32)]),
    "mi_ngram_draft": (C.c_int32, [C.POINTER(C.c_int32), C.c_int32, C.c_int32, C.c_int32, C.POINTER(C.c_int32)]),
    "mi_best_draft_len": (C.c_int32, [C.c_float, C.c_float, C.c_int32]),
    "mi_token_text": (C.c_int32, [_P, C.c_int32, C.c_char_p, C.c_int32]),
    "mi_detok_piece": (C.c_int32, [C.c_char_p, C.c_int32, C.c_char_p, C.c_int32]),
    "mi_teacher": (C.c_int, [_P, C.POINTER(C.c_int32), C.c_int32, C.POINTER(C.c_int32), C.POINTER(C.c_float)]),
    "mi_pred_hash": (C.c_uint64, [C.POINTER(C.c_int32), C.POINTER(C.c_float), C.c_int32]),
    "mi_fnv1a64": (C.c_uint64, [C.c_char_p, C.c_size_t, C.c_uint64]),
}

_lib = None


def lib():
    """Load libminfer.so (raises if it was not built: no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MinferError(-5, "engine library not built: %s (run __graft_entry__.build())" % LIB_PATH)
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(rc, eng=None):
    if rc != MI_OK:
        msg = lib().mi_last_error(eng)
        raise MinferError(rc, msg.decode() if msg else "")


# shapes of BASELINE.json's configs (E, layers, heads/kv, FF, vocab)
SHAPES = {
    "S05": dict(n_layer=24, n_embd=896, n_ff=4864, n_head=14, n_head_kv=2, n_vocab=151936),
    "S15": dict(n_layer=28, n_embd=1536, n_ff=8960, n_head=12, n_head_kv=2, n_vocab=151936),
    "S3": dict(n_layer=36, n_embd=2048, n_ff=11008, n_head=16, n_head_kv=2, n_vocab=151936),
}


GT_Q4_0, GT_Q4_1, GT_Q8_0, GT_Q6_K = 2, 3, 8, 14


def synth_gguf(path, shape, seed, rope_base=1e6, rms_eps=1e-6, emb_q4=False, emb_type=None, head_type=0,
               down_type=0, tied=False, qk_bias_std=0.0, norm_offset=0.0):
    """Write a seeded random-init qwen2 GGUF (mi_synth_gguf). shape: name or dict.
    emb_type 0/2/8 (F32, q4_0, q8_0), head_type 2/8/14 (q4_0, q8_0, q6_K), down_type 2/3
    (q4_0, q4_1), tied: no output.weight (0 means the default of each). qk_bias_std /
    norm_offset: attention scores of order 1 (0 = the BASELINE distributions)."""
    d = SHAPES[shape] if isinstance(shape, str) else shape
    et = emb_type if emb_type is not None else (2 if emb_q4 else 0)
    s = SynthShape(d["n_layer"], d["n_embd"], d["n_ff"], d["n_head"], d["n_head_kv"], d["n_vocab"],
                   rope_base, rms_eps, et, head_type, down_type, 1 if tied else 0, qk_bias_std, norm_offset)
    _check(lib().mi_synth_gguf(path.encode(), C.byref(s), C.c_uint64(seed)))
    return path


def check_layout(shape, max_ctx, n_cu, T, pos):
    """mi_check_layout (host only): (status, message) of the bounds walk of one step"""
    d = SHAPES[shape] if isinstance(shape, str) else shape
    s = SynthShape(d["n_layer"], d["n_embd"], d["n_ff"], d["n_head"], d["n_head_kv"], d["n_vocab"],
                   1e6, 1e-6, 0, 0, 0, 0, 0.0, 0.0)
    buf = C.create_string_buffer(256)
    rc = lib().mi_check_layout(C.byref(s), max_ctx, n_cu, T, pos, buf, 256)
    return rc, buf.value.decode()


def pred_hash(pred, margin):
    """the reference's exactness hash of a teacher-forced run (mi_pred_hash)"""
    n = len(pred)
    assert len(margin) == n
    return lib().mi_pred_hash(_i32(pred), (C.c_float * max(n, 1))(*margin), n)


def fnv1a64(data, basis=14695981039346656037):
    """FNV-1a 64 of a bytes object from `basis` (mi_fnv1a64; default: the published basis)"""
    return lib().mi_fnv1a64(data, len(data), basis)


def default_opts(**kw):
    o = Opts()
    lib().mi_default_opts(C.byref(o))
    for k, v in kw.items():
        setattr(o, k, v)
    return o


def _i32(seq):
    seq = [int(x) for x in seq]
    return (C.c_int32 * max(len(seq), 1))(*seq)


class Engine:
    """One loaded model on one GPU: load / prefill / step / generate."""

    def __init__(self, path, **opts):
        self._h = C.c_void_p()
        o = default_opts(**opts)
        rc = lib().mi_load(path.encode(), C.byref(o), C.byref(self._h))
        _check(rc, None)
        self.info = ModelInfo()
        _check(lib().mi_info(self._h, C.byref(self.info)), self._h)

    def close(self):
        if self._h:
            lib().mi_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def plan(self):
        i = self.info
        return dict(cb=list(i.plan_cb), ks=list(i.plan_ks), attn_chunk=i.attn_chunk, kv_f16=i.kv_f16)

    def prefill(self, ids):
        first, mg = C.c_int32(), C.c_float()
        _check(lib().mi_prefill(self._h, _i32(ids), len(ids), C.byref(first), C.byref(mg)), self._h)
        return first.value, mg.value

    def step(self, tok, pos, want_logits=False):
        """One step at position pos. tok: one token id (returns argmax, margin[,
        logits [V]]) or a list of T <= 8 ids (returns lists, logits [T][V])."""
        many = isinstance(tok, (list, tuple))
        toks = list(tok) if many else [tok]
        T = len(toks)
        am, mg = (C.c_int32 * T)(), (C.c_float * T)()
        lg = (C.c_float * (self.info.n_vocab * T))() if want_logits else None
        _check(lib().mi_step(self._h, _i32(toks), T, pos, am, mg, lg), self._h)
        a, m = (list(am), list(mg)) if many else (am[0], mg[0])
        if want_logits:
            import numpy as np
            l = np.frombuffer(lg, dtype=np.float32).copy()
            return a, m, (l.reshape(T, -1) if many else l)
        return a, m

    def teacher(self, ids):
        """Teacher-forced predictions over ids (mi_teacher): pred[i], margin[i] = the
        greedy prediction after position i (for position i+1) and its margin."""
        n = len(ids)
        pred, mg = (C.c_int32 * n)(), (C.c_float * n)()
        _check(lib().mi_teacher(self._h, _i32(ids), n, pred, mg), self._h)
        return list(pred), list(mg)

    def debug_flag_barrier(self):
        """raise the barrier error flag from the host (test hook of the launch-mode fallback)"""
        _check(lib().mi_debug_flag_barrier(self._h), self._h)

    def refresh_info(self):
        _check(lib().mi_info(self._h, C.byref(self.info)), self._h)
        return self.info

    def generate(self, n_gen, callback=None):
        out = (C.c_int32 * max(n_gen, 1))()
        mg = (C.c_float * max(n_gen, 1))()
        n = C.c_int32()
        cb = TOKEN_CB(lambda t, u: int(bool(callback(t)))) if callback else TOKEN_CB()
        _check(lib().mi_generate(self._h, n_gen, out, mg, C.byref(n), cb, None), self._h)
        return list(out[:n.value]), list(mg[:n.value])

    PHASES = ["qkv", "attn", "attn_comb", "o", "gate_up", "down", "lm_head", "argmax", "step"]

    def time_phase(self, phase, layer=0, reps=20):
        """mean duration (ms) of one phase kernel of the last step, from HIP events"""
        ph = self.PHASES.index(phase) if isinstance(phase, str) else phase
        ms = C.c_double()
        _check(lib().mi_time_phase(self._h, ph, layer, reps, C.byref(ms)), self._h)
        return ms.value

    PROFILE_PHASES = ["qkv", "attn", "o", "gate_up", "down"]
    PROF_PER_PHASE = 8

    @classmethod
    def prof_slot(cls, layer, kind, j):
        """column of stamp j of phase `kind` (0..4; kind 0 of layer n_layer = lm_head)"""
        return 1 + (5 * layer + kind) * cls.PROF_PER_PHASE + j

    def profile_step(self):
        """Stamps of one persistent step: an array [workgroups][1 + 8*(5*n_layer + 1)] of
        microseconds since the earliest start (slot layout in mi_profile_step)."""
        import numpy as np
        nslot = 1 + (5 * self.info.n_layer + 1) * self.PROF_PER_PHASE
        n = nslot * self.info.n_cu
        buf = (C.c_double * n)()
        _check(lib().mi_profile_step(self._h, buf, n), self._h)
        return np.frombuffer(buf, dtype=np.float64).reshape(self.info.n_cu, nslot).copy()

    def profile_summary(self):
        """Per phase, summed over layers (microseconds, (mean, max) over workgroups):
        prep = barrier exit -> prologue end, tiles = -> first worker's tiles done,
        store = -> its stores drained, sync = -> phase end, wait = -> barrier exit;
        barrier = earliest exit minus latest phase end."""
        import numpy as np
        t = self.profile_step()
        L = self.info.n_layer
        out = {}
        parts = ("prep", "tiles", "store", "sync", "wait")
        for k, ph in enumerate(self.PROFILE_PHASES):
            for j, part in enumerate(parts):
                acc = np.zeros(t.shape[0])
                for l in range(L):
                    s = self.prof_slot(l, k, j)
                    prev = s - 1 if j else self.prof_slot(l, k, 0) - self.PROF_PER_PHASE + 4
                    acc += t[:, s] - t[:, prev] if (l, k) != (0, 0) or j else t[:, s] - t[:, 0]
                out[ph + "_" + part] = (round(float(acc.mean()), 1), round(float(acc.max()), 1))
            ends = [self.prof_slot(l, k, 3) for l in range(L)]
            out[ph + "_barrier"] = round(float(sum(t[:, e + 1].min() - t[:, e].max() for e in ends)), 1)
        s0 = self.prof_slot(L, 0, 0)
        for j, part in enumerate(("lm_prep", "lm_tiles", "lm_cand", "lm_sync", "lm_wait")):
            v = t[:, s0 + j] - t[:, s0 + j - 1 if j else s0 - self.PROF_PER_PHASE + 4]
            out[part] = (round(float(v.mean()), 1), round(float(v.max()), 1))
        out["total"] = round(float(t[:, -1].max()), 1)
        return out

    def token_text(self, tok):
        """bytes of one token's text (the GGUF vocab piece, byte-level BPE decoded)"""
        buf = C.create_string_buffer(256)
        n = lib().mi_token_text(self._h, tok, buf, 256)
        if n < 0:
            raise MinferError(n, "token %d outside the vocabulary" % tok)
        if n > 256:
            buf = C.create_string_buffer(n)
            lib().mi_token_text(self._h, tok, buf, n)
        return buf.raw[:n]

    def stats(self):
        s = Stats()
        _check(lib().mi_get_stats(self._h, C.byref(s)), self._h)
        return dict(steps=s.steps, tokens=s.tokens, decode_ms=s.decode_ms, prefill_ms=s.prefill_ms,
                    drafted=s.drafted, accepted=s.accepted)


# ---------------------------------------------------------------- kernel-level helpers
def detok_piece(piece):
    """raw bytes of a byte-level BPE vocab piece (str or UTF-8 bytes)"""
    p = piece.encode("utf-8") if isinstance(piece, str) else bytes(piece)
    cap = len(p) + 1
    buf = C.create_string_buffer(cap)
    n = lib().mi_detok_piece(p, len(p), buf, cap)
    if n < 0:
        raise MinferError(n, "bad piece")
    return buf.raw[:n]


def packed_bytes(rows, nb, cb):
    return lib().mi_q4_packed_bytes(rows, nb, cb)


def pack_q4(src_bytes, rows, nb, cb):
    """GGUF row-major q4_0 bytes (numpy uint8) -> tile layout (numpy uint8)."""
    import numpy as np
    src = np.ascontiguousarray(src_bytes, dtype=np.uint8)
    n = packed_bytes(rows, nb, cb)
    if n == 0 or src.size != rows * nb * 18:
        raise MinferError(-1, "bad q4 matrix shape")
    dst = np.empty(n, dtype=np.uint8)
    _check(lib().mi_q4_pack(src.ctypes.data, rows, nb, cb, dst.ctypes.data))
    return dst


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else C.c_void_p()


def _stream(stream):
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream)


def quant_q8(x, xq, xd, xs8, stream=None):
    _check(lib().mi_quant_q8(_ptr(x), x.numel(), _ptr(xq), _ptr(xd), _ptr(xs8), _stream(stream)))


def gemv_q4(packed, rows, nb, cb, ks, xq, xd, xs8, part, y=None, stream=None):
    _check(lib().mi_gemv_q4(_ptr(packed), rows, nb, cb, ks, _ptr(xq), _ptr(xd), _ptr(xs8), _ptr(part), _ptr(y),
                            _stream(stream)))


def q4_block_isums(packed, rows, nb, cb, xq, isum, stream=None):
    _check(lib().mi_q4_block_isums(_ptr(packed), rows, nb, cb, _ptr(xq), _ptr(isum), _stream(stream)))


def attn_scratch_floats(n_head, hd, L):
    """floats of scratch attn_decode needs for n_head heads of size hd over L positions"""
    return int(lib().mi_attn_scratch_floats(n_head, hd, L))


def attn_decode(q, kc, vc, n_head, n_head_kv, hd, L, ctx, scale, scratch, out, stream=None):
    _check(lib().mi_attn_decode(_ptr(q), _ptr(kc), _ptr(vc), n_head, n_head_kv, hd, L, ctx, C.c_float(scale),
                                _ptr(scratch), _ptr(out), _stream(stream)))


def attn_decode_mfma(q, kc, vc, n_head, n_head_kv, hd, L, ctx, scale, scratch, out, stream=None):
    """attn_decode with MFMA chunk records (mi_attn_decode_mfma): ~1e-6 relative, not bit-identical"""
    _check(lib().mi_attn_decode_mfma(_ptr(q), _ptr(kc), _ptr(vc), n_head, n_head_kv, hd, L, ctx, C.c_float(scale),
                                     _ptr(scratch), _ptr(out), _stream(stream)))


ATTN_NOALLOC_SCRATCH_FLOATS = 4 << 20   # MI_ATTN_NOALLOC_SCRATCH_FLOATS


def attn_decode_noalloc(q, kc, vc, n_head, n_head_kv, hd, L, ctx, scale, out, stream=None):
    """attn_decode with the library's own device scratch (mi_attn_decode_noalloc)"""
    _check(lib().mi_attn_decode_noalloc(_ptr(q), _ptr(kc), _ptr(vc), n_head, n_head_kv, hd, L, ctx,
                                        C.c_float(scale), _ptr(out), _stream(stream)))


def barrier_cost(nwg, n=1000):
    us = C.c_double()
    _check(lib().mi_barrier_cost(nwg, n, C.byref(us)))
    return us.value


def stream_read(buf, nbytes, sink, stream=None):
    _check(lib().mi_stream_read(_ptr(buf), C.c_size_t(nbytes), _ptr(sink), _stream(stream)))


# ---------------------------------------------------------------- seeded inputs
def prompt_ids(seed, n, n_vocab):
    """n token IDs uniform in [0, n_vocab) from a splitmix64 stream (same on any host)."""
    mask = (1 << 64) - 1
    s = (seed * 0x9E3779B97F4A7C15 + 0x632BE59BD9B4E019) & mask
    out = []
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & mask
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        z ^= z >> 31
        out.append(int((z * n_vocab) >> 64))
    return out


# the BASELINE configs as (shape, model seed, prompt seed, prompt length, n_gen)
CONFIGS = {
    "config0": ("S05", 1000, 1001, 16, 128),
    "config2": ("S15", 2000, 2001, 64, 128),
    "config4": ("S3", 4000, 4001, 1024, 8),
}
