"""The engine's C ABI (include/minfer.h) driven through ctypes from a library path: the
HIP library (nano-inference_amd/_build/libminfer.so) or the CPU oracle's implementation
of the same ABI (oracle/_build/liboracle_minfer.so, test infrastructure). The parity
harness runs one call sequence on both and compares what comes back; the same class
drives either, so nothing in the sequence knows which backend it talks to.
"""
import ctypes as C
import os

import numpy as np

import minfer

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIP_LIB = minfer.LIB_PATH
ORACLE_LIB = os.path.join(ROOT, "oracle", "_build", "liboracle_minfer.so")

_I32P = C.POINTER(C.c_int32)
_F32P = C.POINTER(C.c_float)
_SIGS = {
    "mi_default_opts": (None, [C.POINTER(minfer.Opts)]),
    "mi_load": (C.c_int, [C.c_char_p, C.POINTER(minfer.Opts), C.POINTER(C.c_void_p)]),
    "mi_free": (None, [C.c_void_p]),
    "mi_last_error": (C.c_char_p, [C.c_void_p]),
    "mi_info": (C.c_int, [C.c_void_p, C.POINTER(minfer.ModelInfo)]),
    "mi_prefill": (C.c_int, [C.c_void_p, _I32P, C.c_int32, _I32P, _F32P]),
    "mi_step": (C.c_int, [C.c_void_p, _I32P, C.c_int32, C.c_int32, _I32P, _F32P, _F32P]),
    "mi_generate": (C.c_int, [C.c_void_p, C.c_int32, _I32P, _F32P, _I32P, C.c_void_p, C.c_void_p]),
    "mi_teacher": (C.c_int, [C.c_void_p, _I32P, C.c_int32, _I32P, _F32P]),
}
_libs = {}


def backend(path):
    """the library at path with the engine ABI's signatures set"""
    if path not in _libs:
        if not os.path.exists(path):
            raise minfer.MinferError(-5, "library not built: %s" % path)
        L = C.CDLL(path)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _libs[path] = L
    return _libs[path]


def oracle_mode(mode, plan=None):
    """the oracle backend's forward mode (0 fp32, 1 q8act) and q8act plan (cb, ks lists)
    for engines loaded after this call"""
    L = backend(ORACLE_LIB)
    L.orc_mi_set_mode(C.c_int(mode))
    if plan is not None:
        cb = (C.c_int32 * 5)(*plan[0])
        ks = (C.c_int32 * 5)(*plan[1])
        L.orc_mi_set_plan(cb, ks)


def _ints(xs):
    a = np.ascontiguousarray(np.asarray(xs, np.int32))
    return a, a.ctypes.data_as(_I32P)


class AbiEngine:
    def __init__(self, libpath, gguf, **opts):
        self.L = backend(libpath)
        o = minfer.Opts()
        self.L.mi_default_opts(C.byref(o))
        for k, v in opts.items():
            setattr(o, k, v)
        self.h = C.c_void_p()
        self._check(self.L.mi_load(gguf.encode(), C.byref(o), C.byref(self.h)), load=True)
        info = minfer.ModelInfo()
        self._check(self.L.mi_info(self.h, C.byref(info)))
        self.info = info
        self.V = info.n_vocab

    def _check(self, rc, load=False):
        if rc != 0:
            msg = self.L.mi_last_error(None if load else self.h)
            raise minfer.MinferError(rc, msg.decode() if msg else "")

    def close(self):
        if self.h:
            self.L.mi_free(self.h)
            self.h = C.c_void_p()

    def prefill(self, ids):
        a, p = _ints(ids)
        first, mg = C.c_int32(), C.c_float()
        self._check(self.L.mi_prefill(self.h, p, len(a), C.byref(first), C.byref(mg)))
        return first.value, np.float32(mg.value)

    def step(self, toks, pos, want_logits=False):
        a, p = _ints(toks)
        T = len(a)
        am = np.zeros(T, np.int32)
        mg = np.zeros(T, np.float32)
        lg = np.zeros((T, self.V), np.float32) if want_logits else None
        self._check(self.L.mi_step(self.h, p, T, pos, am.ctypes.data_as(_I32P), mg.ctypes.data_as(_F32P),
                                   lg.ctypes.data_as(_F32P) if want_logits else None))
        return am, mg, lg

    def generate(self, n):
        out = np.zeros(max(n, 1), np.int32)
        mg = np.zeros(max(n, 1), np.float32)
        got = C.c_int32()
        self._check(self.L.mi_generate(self.h, n, out.ctypes.data_as(_I32P), mg.ctypes.data_as(_F32P),
                                       C.byref(got), None, None))
        return out[:got.value], mg[:got.value]

    def teacher(self, ids):
        a, p = _ints(ids)
        pred = np.zeros(len(a), np.int32)
        mg = np.zeros(len(a), np.float32)
        self._check(self.L.mi_teacher(self.h, p, len(a), pred.ctypes.data_as(_I32P), mg.ctypes.data_as(_F32P)))
        return pred, mg


def session(eng, prompt, n_gen, step_toks):
    """one call sequence, the same for every backend: prefill, generate, a multi-token
    step with logits at the end of the context, then teacher forcing over the whole
    sequence. Returns everything that came back."""
    first, m0 = eng.prefill(prompt)
    toks, mg = eng.generate(n_gen)
    pos = len(prompt) + n_gen - 1
    am, smg, lg = eng.step(step_toks, pos, want_logits=True)
    seq = list(prompt) + [int(t) for t in toks]
    pred, tmg = eng.teacher(seq)
    return dict(first=first, m0=m0, toks=toks, mg=mg, step_argmax=am, step_margin=smg, step_logits=lg, pred=pred,
                teacher_margin=tmg)
