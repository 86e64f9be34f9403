"""ctypes binding of the CPU oracle (oracle/_build/liboracle.so) for the tests.

The oracle is test infrastructure: only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py load it, as the checker (or the timed CPU baseline).
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "_build", "liboracle.so")
REF_BIN = os.path.join(ROOT, "oracle", "_ref", "cpu_infer")
MODE_FP32, MODE_Q8ACT = 0, 1


class Plan(C.Structure):
    _fields_ = [("cb", C.c_int32 * 5), ("ks", C.c_int32 * 5), ("attn_chunk", C.c_int32), ("kv_f16", C.c_int32)]

    @staticmethod
    def make(cb, ks, attn_chunk=64, kv_f16=1):
        p = Plan()
        for i in range(5):
            p.cb[i] = cb[i]
            p.ks[i] = ks[i]
        p.attn_chunk = attn_chunk
        p.kv_f16 = kv_f16
        return p


class Config(C.Structure):
    _fields_ = [("n_layer", C.c_int32), ("n_embd", C.c_int32), ("n_ff", C.c_int32), ("n_head", C.c_int32),
                ("n_head_kv", C.c_int32), ("head_dim", C.c_int32), ("n_vocab", C.c_int32),
                ("rope_base", C.c_float), ("rms_eps", C.c_float)]


_P = C.c_void_p
_F = C.POINTER(C.c_float)
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError("oracle not built: %s (make -C oracle)" % LIB)
        L = C.CDLL(LIB)
        sig = {
            "orc_gguf_open": (_P, [C.c_char_p]),
            "orc_gguf_close": (None, [_P]),
            "orc_gguf_error": (C.c_char_p, []),
            "orc_gguf_num": (C.c_double, [_P, C.c_char_p, C.c_double]),
            "orc_gguf_n_tokens": (C.c_int64, [_P]),
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_expf": (C.c_float, [C.c_float]),
            "orc_quant_q8": (None, [_P, C.c_int, _P, _P, _P]),
            "orc_q4_block_isum": (C.c_int32, [_P, _P]),
            "orc_q4_row_dot": (C.c_float, [_P, C.c_int, C.c_int, C.c_int, _P, _P, _P]),
            "orc_rmsnorm_canon": (None, [_P, _P, C.c_int, C.c_float, _P]),
            "orc_butterfly64": (C.c_float, [_P]),
            "orc_model_new": (_P, [_P, C.c_int, C.POINTER(Plan), C.c_int, C.c_int]),
            "orc_model_free": (None, [_P]),
            "orc_model_config": (None, [_P, C.POINTER(Config)]),
            "orc_forward": (C.c_int32, [_P, C.c_int32, C.c_int32, _P, _F]),
            "orc_generate": (C.c_int, [_P, _P, C.c_int32, C.c_int32, _P, _P, C.POINTER(C.c_double),
                                       C.POINTER(C.c_double)]),
            "orc_attention_canon": (None, [_P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int, _P]),
            "orc_attention_fp32": (None, [_P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_float, _P]),
            "orc_rope_cs": (None, [C.c_int, C.c_int, C.c_int, C.c_float, _F, _F]),
            "orc_rope_rotate": (None, [_P, C.c_int, C.c_int, _P, _P]),
            "orc_rope_fp32": (None, [_P, C.c_int, C.c_int, C.c_int, C.c_float]),
            "orc_dequant_row": (None, [_P, C.c_int64, _P]),
            "orc_dequant_row_fma": (None, [_P, C.c_int64, _P]),
            "orc_requant_q4_0_row": (None, [_P, C.c_int, _P]),
        }
        for k, (r, a) in sig.items():
            f = getattr(L, k)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def ptr(a):
    return C.c_void_p(a.ctypes.data)


def expf(x):
    return lib().orc_expf(C.c_float(x))


def quant_q8(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.size
    xq = np.zeros(n, np.int8)
    xd = np.zeros(n // 32, np.float32)
    xs8 = np.zeros(n // 32, np.int32)
    lib().orc_quant_q8(ptr(x), n, ptr(xq), ptr(xd), ptr(xs8))
    return xq, xd, xs8


def row_dot(row_bytes, nb, cb, ks, xq, xd, xs8):
    row_bytes = np.ascontiguousarray(row_bytes, dtype=np.uint8)
    return lib().orc_q4_row_dot(ptr(row_bytes), nb, cb, ks, ptr(xq), ptr(xd), ptr(xs8))


def rmsnorm_canon(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros_like(x)
    lib().orc_rmsnorm_canon(ptr(x), ptr(w), x.size, C.c_float(eps), ptr(out))
    return out


def attention_canon(q, k, v, L, hd, stride, scale):
    out = np.zeros(hd, np.float32)
    lib().orc_attention_canon(ptr(q), ptr(k), ptr(v), L, hd, stride, C.c_float(scale), 64, ptr(out))
    return out


def attention_fp32(q, k, v, L, hd, stride, scale):
    out = np.zeros(hd, np.float32)
    lib().orc_attention_fp32(ptr(q), ptr(k), ptr(v), L, hd, stride, C.c_float(scale), ptr(out))
    return out


def rope_rotate(v, n_head, hd, c, s):
    """the q8act mode's NEOX rotation (orc_rope_rotate) of a copy of v [n_head*hd]"""
    v = np.array(v, dtype=np.float32)
    c = np.ascontiguousarray(c, dtype=np.float32)
    s = np.ascontiguousarray(s, dtype=np.float32)
    lib().orc_rope_rotate(ptr(v), n_head, hd, ptr(c), ptr(s))
    return v


def rope_fp32(v, n_head, hd, pos, base):
    """the fp32 mode's RoPE (orc_rope_fp32, cpu_infer.cpp:49-61) of a copy of v"""
    v = np.array(v, dtype=np.float32)
    lib().orc_rope_fp32(ptr(v), n_head, hd, pos, C.c_float(base))
    return v


def rope_cs(pos, hd, base):
    """cos/sin of every pair at position pos as cpu_infer computes them"""
    c = np.zeros(hd // 2, np.float32)
    s = np.zeros(hd // 2, np.float32)
    for i in range(hd // 2):
        cc, ss = C.c_float(), C.c_float()
        lib().orc_rope_cs(pos, i, hd, C.c_float(base), C.byref(cc), C.byref(ss))
        c[i], s[i] = cc.value, ss.value
    return c, s


class Model:
    """oracle model over a GGUF: mode MODE_FP32 (cpu_infer) or MODE_Q8ACT (engine numerics)."""

    def __init__(self, path, mode, plan=None, max_seq=512, threads=0):
        L = lib()
        self.g = L.orc_gguf_open(path.encode())
        if not self.g:
            raise RuntimeError("oracle gguf: %s" % L.orc_gguf_error().decode())
        p = C.byref(plan) if plan is not None else None
        self.m = L.orc_model_new(self.g, mode, p, max_seq, threads)
        if not self.m:
            raise RuntimeError("oracle model setup failed")
        self.cfg = Config()
        L.orc_model_config(self.m, C.byref(self.cfg))

    def forward(self, tok, pos, want_logits=False):
        lg = np.zeros(self.cfg.n_vocab, np.float32) if want_logits else None
        mg = C.c_float()
        r = lib().orc_forward(self.m, tok, pos, ptr(lg) if lg is not None else None, C.byref(mg))
        if r < 0:
            raise RuntimeError("oracle forward failed")
        return (r, mg.value, lg) if want_logits else (r, mg.value)

    def generate(self, prompt, n_gen):
        pr = np.asarray(prompt, np.int32)
        out = np.zeros(max(n_gen, 1), np.int32)
        mg = np.zeros(max(n_gen, 1), np.float32)
        tp, td = C.c_double(), C.c_double()
        if lib().orc_generate(self.m, ptr(pr), len(pr), n_gen, ptr(out), ptr(mg), C.byref(tp), C.byref(td)):
            raise RuntimeError("oracle generate failed")
        return out[:n_gen].tolist(), mg[:n_gen].tolist(), tp.value, td.value

    def close(self):
        if self.m:
            lib().orc_model_free(self.m)
            self.m = None
        if self.g:
            lib().orc_gguf_close(self.g)
            self.g = None

    def __del__(self):
        self.close()
