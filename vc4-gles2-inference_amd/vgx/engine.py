"""ctypes binding of the decode engine (include/vgx_engine.h)."""
import ctypes
import os

import numpy as np

from . import lib as _l

# VGX_ENGINE_LIB names another build of the engine library; by default the
# in-tree build.
LIB_PATH = os.environ.get("VGX_ENGINE_LIB") or os.path.join(_l.PKG, "lib", "libvgx_engine.so")
CLI_PATH = os.path.join(_l.PKG, "bin", "engine_mm3")

_P = ctypes.c_void_p
_I = ctypes.c_int
_SIGS = {
    "vgx_engine_open": (_I, [ctypes.c_char_p, _I, _I, _I, ctypes.POINTER(_P)]),
    "vgx_engine_open_bytes": (_I, [_P, ctypes.c_size_t, _I, _I, _I, ctypes.POINTER(_P)]),
    "vgx_engine_close": (_I, [_P]),
    "vgx_engine_info": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "vgx_engine_step": (_I, [_P, _I, _I, _P, ctypes.POINTER(_I)]),
    "vgx_engine_generate": (_I, [_P, _P, _I, _I, _P, ctypes.POINTER(ctypes.c_double),
                                 ctypes.POINTER(ctypes.c_double)]),
    "vgx_engine_prefill": (_I, [_P, _P, _I, _I, _P, ctypes.POINTER(_I)]),
    "vgx_engine_set_prefill_batch": (_I, [_P, _I]),
    "vgx_engine_generate_batch": (_I, [_P, _I, _P, _I, _I, _P, ctypes.POINTER(ctypes.c_double),
                                       ctypes.POINTER(ctypes.c_double)]),
    "vgx_engine_generate_from": (_I, [_P, _P, _I, _I, _I, _P, ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(ctypes.c_double)]),
    "vgx_engine_save_prefix": (_I, [_P, ctypes.c_char_p, _P, _I, ctypes.c_uint64, ctypes.c_uint64]),
    "vgx_engine_conv_layers": (_I, [_P]),
    "vgx_engine_set_graphs": (_I, [_P, _I]),
    "vgx_engine_load_prefix": (_I, [_P, ctypes.c_char_p, _P, _I, ctypes.POINTER(_I)]),
    "vgx_engine_step_candidates": (_I, [_P, _I, _I, _I, ctypes.c_float, ctypes.c_float, _P, _P, _I,
                                        ctypes.POINTER(_I), _P, ctypes.POINTER(_I), _P]),
    "vgx_sampler_create": (_I, [ctypes.c_uint32, ctypes.POINTER(_P)]),
    "vgx_sampler_free": (_I, [_P]),
    "vgx_sample_logits": (_I, [_P, _P, _I, ctypes.c_float, ctypes.c_float, _I, ctypes.POINTER(_I),
                               ctypes.POINTER(ctypes.c_float)]),
    "vgx_argmax_report": (_I, [_P, _I, ctypes.POINTER(_I), ctypes.POINTER(ctypes.c_float)]),
    "vgx_sample_candidates": (_I, [_P, _P, _P, _I, _I, ctypes.c_float, ctypes.c_float, ctypes.c_float, _I,
                                   ctypes.POINTER(_I)]),
    "vgx_apply_penalties": (_I, [_P, _I, _P, _I, ctypes.c_float, ctypes.c_float, ctypes.c_float, _I,
                                 ctypes.c_float]),
    "vgx_engine_last_error": (ctypes.c_char_p, []),
}
_lib = None


def load():
    global _lib
    if _lib is None:
        _l.load()  # libvgx first: the engine links it
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("libvgx_engine is not built (%s)" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            getattr(L, name).restype = res
            getattr(L, name).argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return sorted(_SIGS)


def _check(st):
    if st != 0:
        raise _l.VgxError(st, load().vgx_engine_last_error().decode())


class Engine:
    """An MMCF model on one GPU: step (Session::step) and greedy generate."""

    def __init__(self, blob=None, path=None, device=0, seq=0, kv_bits=16):
        L = load()
        h = ctypes.c_void_p()
        if path is not None:
            _check(L.vgx_engine_open(path.encode(), device, seq, kv_bits, ctypes.byref(h)))
            self._blob = None
        else:
            self._blob = np.frombuffer(blob, np.uint8).copy()  # the engine borrows it until close
            _check(L.vgx_engine_open_bytes(self._blob.ctypes.data, self._blob.size, device, seq, kv_bits,
                                           ctypes.byref(h)))
        self.h = h
        d, l, v, s = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        _check(L.vgx_engine_info(h, ctypes.byref(d), ctypes.byref(l), ctypes.byref(v), ctypes.byref(s)))
        self.dim, self.layers, self.vocab, self.seq = d.value, l.value, v.value, s.value

    def step(self, token, pos, logits=True):
        out = np.empty(self.vocab, np.int16) if logits else None
        nx = ctypes.c_int()
        _check(load().vgx_engine_step(self.h, int(token), int(pos),
                                      ctypes.c_void_p(out.ctypes.data if logits else 0), ctypes.byref(nx)))
        return out, nx.value

    def prefill(self, tokens, pos0=0, logits=True):
        """Positions pos0.. of `tokens` in batches; the last one's logits and argmax."""
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.vocab, np.int16) if logits else None
        nx = ctypes.c_int()
        _check(load().vgx_engine_prefill(self.h, t.ctypes.data, t.size, int(pos0),
                                         ctypes.c_void_p(out.ctypes.data if logits else 0), ctypes.byref(nx)))
        return out, nx.value

    def set_graphs(self, on):
        """Decode steps as one replayed HIP graph (True) or single launches."""
        _check(load().vgx_engine_set_graphs(self.h, int(bool(on))))

    def set_prefill_batch(self, n):
        """Largest prompt batch (0 or 1: one position at a time)."""
        _check(load().vgx_engine_set_prefill_batch(self.h, int(n)))

    def generate(self, prompt, n_gen):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_gen, np.int32)
        pf, dc = ctypes.c_double(), ctypes.c_double()
        _check(load().vgx_engine_generate(self.h, p.ctypes.data, p.size, n_gen, out.ctypes.data,
                                          ctypes.byref(pf), ctypes.byref(dc)))
        return out, pf.value, dc.value

    def generate_from(self, prompt, n_cached, n_gen):
        """generate() with prompt[:n_cached] already in the KV cache."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_gen, np.int32)
        pf, dc = ctypes.c_double(), ctypes.c_double()
        _check(load().vgx_engine_generate_from(self.h, p.ctypes.data, p.size, n_cached, n_gen, out.ctypes.data,
                                               ctypes.byref(pf), ctypes.byref(dc)))
        return out, pf.value, dc.value

    def save_prefix(self, path, toks, system_fnv=0, tools_fnv=0):
        """The MMKV1 cache of positions 0..len(toks)-1 (and its .json sidecar)."""
        t = np.ascontiguousarray(toks, np.int32)
        _check(load().vgx_engine_save_prefix(self.h, str(path).encode(), t.ctypes.data, t.size, system_fnv,
                                             tools_fnv))

    def load_prefix(self, path):
        """Load an MMKV1 cache; returns its token ids."""
        n = ctypes.c_int()
        buf = np.empty(self.seq, np.int32)
        _check(load().vgx_engine_load_prefix(self.h, str(path).encode(), buf.ctypes.data, buf.size,
                                             ctypes.byref(n)))
        return buf[:n.value].copy()

    def step_candidates(self, token, pos, topk, temp, top_p):
        """One position's top-k candidates (Session::step_candidates): a dict
        with values, tokens, logsumexp, max_logit, denom, complete and, when
        not complete, the full float logits."""
        value = np.empty(topk, np.float32)
        tok = np.empty(topk, np.int32)
        full = np.empty(self.vocab, np.float32)
        stats = np.empty(3, np.float32)
        n, comp = ctypes.c_int(), ctypes.c_int()
        _check(load().vgx_engine_step_candidates(self.h, int(token), int(pos), int(topk), float(temp), float(top_p),
                                                 value.ctypes.data, tok.ctypes.data, topk, ctypes.byref(n),
                                                 stats.ctypes.data, ctypes.byref(comp), full.ctypes.data))
        k = n.value
        return {"values": value[:k].copy(), "tokens": tok[:k].copy(), "logsumexp": float(stats[0]),
                "max_logit": float(stats[1]), "denom": float(stats[2]), "complete": bool(comp.value),
                "full": None if comp.value else full}

    def generate_batch(self, prompts, n_gen):
        """Greedy generation for the rows of prompts (nseq x n_prompt) in
        lockstep: (nseq x n_gen tokens, prefill_ms, decode_ms)."""
        p = np.ascontiguousarray(prompts, np.int32)
        nseq, n_prompt = p.shape
        out = np.empty((nseq, n_gen), np.int32)
        pf, dc = ctypes.c_double(), ctypes.c_double()
        _check(load().vgx_engine_generate_batch(self.h, nseq, p.ctypes.data, n_prompt, n_gen, out.ctypes.data,
                                                ctypes.byref(pf), ctypes.byref(dc)))
        return out, pf.value, dc.value

    def close(self):
        if self.h:
            load().vgx_engine_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Sampler:
    """The host sampler (engine/src/sampling.cpp) with its own std::mt19937."""

    def __init__(self, seed):
        h = ctypes.c_void_p()
        _check(load().vgx_sampler_create(ctypes.c_uint32(seed & 0xFFFFFFFF), ctypes.byref(h)))
        self.h = h

    def sample_logits(self, logits, temp, top_p, top_k=0):
        """(token, log-probability within the kept set)."""
        x = np.ascontiguousarray(logits, np.float32)
        t, lp = ctypes.c_int(), ctypes.c_float()
        _check(load().vgx_sample_logits(self.h, x.ctypes.data, x.size, float(temp), float(top_p), int(top_k),
                                        ctypes.byref(t), ctypes.byref(lp)))
        return t.value, lp.value

    def sample_candidates(self, values, tokens, strict, logsumexp, temp, top_p, top_k):
        v = np.ascontiguousarray(values, np.float32)
        k = np.ascontiguousarray(tokens, np.int32)
        t = ctypes.c_int()
        _check(load().vgx_sample_candidates(self.h, v.ctypes.data, k.ctypes.data, v.size, int(bool(strict)),
                                            float(logsumexp), float(temp), float(top_p), int(top_k),
                                            ctypes.byref(t)))
        return t.value

    def close(self):
        if self.h:
            load().vgx_sampler_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def argmax_report(logits):
    x = np.ascontiguousarray(logits, np.float32)
    t, lp = ctypes.c_int(), ctypes.c_float()
    _check(load().vgx_argmax_report(x.ctypes.data, x.size, ctypes.byref(t), ctypes.byref(lp)))
    return t.value, lp.value


def apply_penalties(logits, recent, repetition=1.0, frequency=0.0, presence=0.0, no_repeat_ngram=0, min_p=0.0):
    """apply_sampling_penalties on a copy of logits."""
    x = np.array(logits, np.float32)
    r = np.ascontiguousarray(recent, np.int32)
    _check(load().vgx_apply_penalties(x.ctypes.data, x.size, r.ctypes.data if r.size else None, r.size,
                                      float(repetition), float(frequency), float(presence), int(no_repeat_ngram),
                                      float(min_p)))
    return x
