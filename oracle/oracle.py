"""numpy front end of the C oracle (oracle/vgx_oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, the smoke check and bench.py's cpu_baseline
leg import this module, as the checker or as the timed CPU baseline; the
product never does.  Each function names the reference file:line it restates
(paths relative to the reference repository root).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "lib", "libvgx_oracle.so")

_c_i16 = np.ctypeslib.ndpointer(np.int16, flags="C")
_c_i8 = np.ctypeslib.ndpointer(np.int8, flags="C")
_c_u8 = np.ctypeslib.ndpointer(np.uint8, flags="C")
_c_f32 = np.ctypeslib.ndpointer(np.float32, flags="C")
_c_i32 = np.ctypeslib.ndpointer(np.int32, flags="C")
_c_i64 = np.ctypeslib.ndpointer(np.int64, flags="C")
_vp = ctypes.c_void_p
_i = ctypes.c_int
_l = ctypes.c_long
_f = ctypes.c_float
_d = ctypes.POINTER(ctypes.c_double)


class AttnCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in
                ("dim", "heads", "kv_heads", "head_dim", "seq", "kv_bits", "rope_half", "qk_norm")]


def _load():
    if not os.path.exists(_LIB):
        raise RuntimeError("oracle library missing: run `make -C oracle` (%s)" % _LIB)
    L = ctypes.CDLL(_LIB)
    sig = {
        "vgxo_quantize_act": (ctypes.c_int16, [_f]),
        "vgxo_quantize_act_n": (None, [_c_f32, _l, _c_i16]),
        "vgxo_x_texels": (_i, [_i, _i]),
        "vgxo_x_pack": (None, [_c_f32, _i, _i, _c_u8]),
        "vgxo_q16_store": (ctypes.c_int16, [_f]),
        "vgxo_q16_round": (ctypes.c_int16, [_f]),
        "vgxo_qmat": (None, [_c_f32, _l, _c_i16, _d]),
        "vgxo_q8mat": (None, [_c_f32, _l, _c_i8, _d]),
        "vgxo_q8_from_i16": (None, [_c_f32, _l, _c_i8, _d]),
        "vgxo_q8_per_row": (None, [_c_f32, _i, _i, _c_i8, ctypes.POINTER(_f), _c_f32]),
        "vgxo_q4mat": (_i, [_c_f32, _i, _i, _c_u8, _c_i16, _c_i16, _d]),
        "vgxo_t3mat": (_i, [_c_f32, _i, _i, _c_u8, ctypes.POINTER(_f), _c_f32]),
        "vgxo_t3_codes": (None, [_c_u8, _i, _i, _c_u8]),
        "vgxo_t3_bytes": (_l, [_i, _i]),
        "vgxo_row_scales": (None, [_i, _f, _vp, _c_f32]),
        "vgxo_dequant_q8": (None, [_c_u8, _i, _i, _i, _c_f32, _c_f32]),
        "vgxo_dequant_q4": (None, [_c_u8, _c_i16, _c_i16, _f, _i, _i, _c_f32]),
        "vgxo_dequant_t3": (None, [_c_u8, _i, _i, _c_f32, _c_f32]),
        "vgxo_rowval_q8": (None, [_c_u8, _i, _i, _i, _c_f32, _c_i16, _c_f32]),
        "vgxo_rowval_q8_ref32": (None, [_c_u8, _i, _i, _i, _c_f32, _c_i16, _c_f32]),
        "vgxo_rowsum_q8": (None, [_c_u8, _i, _i, _i, _c_i16, _c_i64]),
        "vgxo_rowval_q4": (None, [_c_u8, _c_i16, _c_i16, _f, _i, _i, _c_i16, _c_f32]),
        "vgxo_rowval_q4_ref32": (None, [_c_u8, _c_i16, _c_i16, _f, _i, _i, _c_i16, _c_f32]),
        "vgxo_rowval_t3": (None, [_c_u8, _i, _i, _c_f32, _c_i16, _c_f32]),
        "vgxo_rowval_t3_ref32": (None, [_c_u8, _i, _i, _c_f32, _c_i16, _c_f32]),
        "vgxo_store": (None, [_c_f32, _vp, _i, _c_i16]),
        "vgxo_store_f32": (None, [_c_f32, _i, _c_f32]),
        "vgxo_gate": (None, [_c_f32, _c_f32, _i, _i, _c_i16]),
        "vgxo_probe_q8": (None, [_c_i8, _i, _i, _vp, _f, _c_i16, _vp, _c_i32]),
        "vgxo_rmsnorm": (None, [_c_i16, _c_i16, _i, _f, _c_i16]),
        "vgxo_rmsnorm_stats": (None, [_c_i16, _i, _c_i64, _c_i64]),
        "vgxo_rope_table": (None, [_c_f32, _c_f32, _i, _i, _c_i32]),
        "vgxo_rope_cos_sin": (None, [_f, _i, _i, _c_f32, _c_f32]),
        "vgxo_kv_row_bytes": (_i, [ctypes.POINTER(AttnCfg)]),
        "vgxo_kv_write": (None, [ctypes.POINTER(AttnCfg), _c_i16, _vp, _c_i32, _i, _c_u8]),
        "vgxo_q_rot": (None, [ctypes.POINTER(AttnCfg), _c_i16, _vp, _c_i32, _i, _c_i16]),
        "vgxo_attn_scores": (None, [ctypes.POINTER(AttnCfg), _c_i16, _c_u8, _i, _c_i16]),
        "vgxo_attn_stats": (None, [ctypes.POINTER(AttnCfg), _c_i16, _i, _c_i16]),
        "vgxo_attn_v": (None, [ctypes.POINTER(AttnCfg), _c_i16, _c_i16, _c_u8, _i, _c_i16]),
        "vgxo_attn_block": (None, [ctypes.POINTER(AttnCfg), _c_i16, _vp, _vp, _c_i32, _i, _c_u8, _c_i16]),
        "vgxo_kv_decode": (_f, [ctypes.POINTER(AttnCfg), _c_u8, _i]),
        "vgxo_embed_q8": (None, [_c_i8, _c_f32, _i, _i, _c_i16]),
        "vgxo_conv_taps": (None, [_c_f32, _i, _i, _c_i16]),
        "vgxo_conv_step": (None, [_i, _c_i16, _c_i16, _c_i16, _c_i16, _c_i16]),
        "vgxo_argmax_i16": (_i, [_c_i16, _i]),
        "vgxo_matvec_f32": (None, [_c_f32, _i, _i, _c_f32, _c_f32]),
        "vgxo_rms_f32": (None, [_c_f32, _vp, _i, _f, _c_f32]),
        "vgxo_threads": (_i, []),
        "vgxo_set_threads": (None, [_i]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


lib = _load()


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---- activation grid -------------------------------------------------------
I16_1, I16_2, I8_4, I24_1, F32, BF16 = range(6)


def quantize_act(v):
    """quantize_act (engine/src/common.h:188-195) over an array."""
    v = _c(v, np.float32).ravel()
    out = np.empty(v.size, np.int16)
    lib.vgxo_quantize_act_n(v, v.size, out)
    return out


def x_pack(values, fmt):
    """x_pack (engine/src/xformat.cpp:45-104): texel bytes."""
    v = _c(values, np.float32).ravel()
    out = np.zeros(4 * max(lib.vgxo_x_texels(v.size, fmt), 0), np.uint8)
    if v.size:
        lib.vgxo_x_pack(v, v.size, fmt, out)
    return out


# ---- packers (engine/tools/mmcf_hf.py) -------------------------------------
def qmat(w):
    w = _c(w, np.float32)
    q = np.empty(w.shape, np.int16)
    s = ctypes.c_double()
    lib.vgxo_qmat(w.ravel(), w.size, q.ravel(), ctypes.byref(s))
    return q, s.value


def q8mat(w):
    w = _c(w, np.float32)
    q = np.empty(w.shape, np.int8)
    s = ctypes.c_double()
    lib.vgxo_q8mat(w.ravel(), w.size, q.reshape(-1), ctypes.byref(s))
    return q, s.value


def q8_from_i16(w):
    w = _c(w, np.float32)
    q = np.empty(w.shape, np.int8)
    s = ctypes.c_double()
    lib.vgxo_q8_from_i16(w.ravel(), w.size, q.reshape(-1), ctypes.byref(s))
    return q, s.value


def q8_per_row(w):
    w = _c(w, np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    plane = np.empty(rows, np.float32)
    unit = ctypes.c_float()
    lib.vgxo_q8_per_row(w, rows, cols, q, ctypes.byref(unit), plane)
    return q, unit.value, plane


def q4mat(w):
    w = _c(w, np.float32)
    rows, cols = w.shape
    packed = np.empty((rows, cols // 2), np.uint8)
    s16 = np.empty((rows, cols // 32), np.int16)
    m16 = np.empty((rows, cols // 32), np.int16)
    ps = ctypes.c_double()
    if lib.vgxo_q4mat(w, rows, cols, packed, s16, m16, ctypes.byref(ps)) != 0:
        raise ValueError("q4 cols must be divisible by 32")
    return packed, s16, m16, ps.value


def t3_bytes(rows, cols):
    return int(lib.vgxo_t3_bytes(rows, cols))


def t3mat(w):
    w = _c(w, np.float32)
    rows, cols = w.shape
    packed = np.empty(t3_bytes(rows, cols), np.uint8)
    plane = np.empty(rows, np.float32)
    unit = ctypes.c_float()
    rc = lib.vgxo_t3mat(w, rows, cols, packed, ctypes.byref(unit), plane)
    if rc != 0:
        raise ValueError("t3mat: not per-row ternary (%d)" % rc)
    return packed, unit.value, plane


def t3_codes(packed, rows, cols):
    out = np.empty((rows, cols), np.uint8)
    lib.vgxo_t3_codes(_c(packed, np.uint8), rows, cols, out)
    return out


# ---- unpack / dequantise -----------------------------------------------------
def row_scales(rows, scale, plane=None):
    out = np.empty(rows, np.float32)
    p = None if plane is None else _c(plane, np.float32)
    lib.vgxo_row_scales(rows, scale, _ptr(p), out)
    return out


def dequant_q8(body, prebiased, rows, cols, wsr):
    out = np.empty((rows, cols), np.float32)
    lib.vgxo_dequant_q8(_c(body, np.uint8).ravel(), int(prebiased), rows, cols, _c(wsr, np.float32), out)
    return out


def dequant_q4(nib, s16, m16, ps, rows, cols):
    out = np.empty((rows, cols), np.float32)
    lib.vgxo_dequant_q4(_c(nib, np.uint8).ravel(), _c(s16, np.int16).ravel(), _c(m16, np.int16).ravel(),
                        ps, rows, cols, out)
    return out


def dequant_t3(body, rows, cols, wsr):
    out = np.empty((rows, cols), np.float32)
    lib.vgxo_dequant_t3(_c(body, np.uint8).ravel(), rows, cols, _c(wsr, np.float32), out)
    return out


# ---- GEMV row values and stores ----------------------------------------------
def rowval_q8(body, prebiased, rows, cols, wsr, x, ref32=False):
    out = np.empty(rows, np.float32)
    fn = lib.vgxo_rowval_q8_ref32 if ref32 else lib.vgxo_rowval_q8
    fn(_c(body, np.uint8).ravel(), int(prebiased), rows, cols, _c(wsr, np.float32), _c(x, np.int16), out)
    return out


def rowsum_q8(body, prebiased, rows, cols, x):
    out = np.empty(rows, np.int64)
    lib.vgxo_rowsum_q8(_c(body, np.uint8).ravel(), int(prebiased), rows, cols, _c(x, np.int16), out)
    return out


def rowval_q4(nib, s16, m16, ps, rows, cols, x, ref32=False):
    out = np.empty(rows, np.float32)
    fn = lib.vgxo_rowval_q4_ref32 if ref32 else lib.vgxo_rowval_q4
    fn(_c(nib, np.uint8).ravel(), _c(s16, np.int16).ravel(), _c(m16, np.int16).ravel(), ps, rows, cols,
       _c(x, np.int16), out)
    return out


def rowval_t3(body, rows, cols, wsr, x, ref32=False):
    out = np.empty(rows, np.float32)
    fn = lib.vgxo_rowval_t3_ref32 if ref32 else lib.vgxo_rowval_t3
    fn(_c(body, np.uint8).ravel(), rows, cols, _c(wsr, np.float32), _c(x, np.int16), out)
    return out


def store(v, res=None):
    v = _c(v, np.float32)
    out = np.empty(v.size, np.int16)
    r = None if res is None else _c(res, np.int16)
    lib.vgxo_store(v, _ptr(r), v.size, out)
    return out


def store_f32(v):
    v = _c(v, np.float32)
    out = np.empty(v.size, np.float32)
    lib.vgxo_store_f32(v, v.size, out)
    return out


def gate(v1, v3, hs=0):
    v1 = _c(v1, np.float32)
    out = np.empty(v1.size, np.int16)
    lib.vgxo_gate(v1, _c(v3, np.float32), v1.size, hs, out)
    return out


def probe_q8(w_signed, srow, unit, xq, res=None):
    w_signed = _c(w_signed, np.int8)
    rows, cols = w_signed.shape
    out = np.empty(rows, np.int32)
    s = None if srow is None else _c(srow, np.float32)
    r = None if res is None else _c(res, np.int16)
    lib.vgxo_probe_q8(w_signed, rows, cols, _ptr(s), unit, _c(xq, np.int16), _ptr(r), out)
    return out


def rmsnorm(x, w, eps=1e-5):
    x = _c(x, np.int16)
    out = np.empty(x.size, np.int16)
    lib.vgxo_rmsnorm(x, _c(w, np.int16), x.size, eps, out)
    return out


def rmsnorm_stats(x):
    x = _c(x, np.int16)
    parts = np.empty(32, np.int64)
    tot = np.empty(1, np.int64)
    lib.vgxo_rmsnorm_stats(x, x.size, parts, tot)
    return parts, int(tot[0])


# ---- attention ------------------------------------------------------------------
def attn_cfg(dim, heads, kv_heads, head_dim, seq, kv_bits=16, rope_half=1, qk_norm=1):
    return AttnCfg(dim, heads, kv_heads, head_dim, seq, kv_bits, rope_half, qk_norm)


def rope_cos_sin(theta, head_dim, seq):
    half = head_dim // 2
    c = np.empty((seq, half), np.float32)
    s = np.empty((seq, half), np.float32)
    lib.vgxo_rope_cos_sin(theta, head_dim, seq, c, s)
    return c, s


def rope_table(rcos, rsin):
    seq, half = rcos.shape
    out = np.empty((seq, half, 2), np.int32)
    lib.vgxo_rope_table(_c(rcos, np.float32), _c(rsin, np.float32), seq, half, out)
    return out


def kv_row_bytes(cfg):
    return lib.vgxo_kv_row_bytes(ctypes.byref(cfg))


def kv_write(cfg, qkv, kn, rtab, pos, kv):
    row = np.zeros(kv_row_bytes(cfg), np.uint8)
    lib.vgxo_kv_write(ctypes.byref(cfg), _c(qkv, np.int16), _ptr(None if kn is None else _c(kn, np.int16)),
                      _c(rtab, np.int32), pos, row)
    kv[pos * row.size:(pos + 1) * row.size] = row
    return row


def kv_decode(cfg, row):
    """decKV of every value of one texel row: K values then V values."""
    row = _c(row, np.uint8)
    n = 2 * cfg.kv_heads * cfg.head_dim
    return np.array([lib.vgxo_kv_decode(ctypes.byref(cfg), row, i) for i in range(n)], np.float64)


def q_rot(cfg, qkv, qn, rtab, pos):
    out = np.empty(cfg.dim, np.int16)
    lib.vgxo_q_rot(ctypes.byref(cfg), _c(qkv, np.int16), _ptr(None if qn is None else _c(qn, np.int16)),
                   _c(rtab, np.int32), pos, out)
    return out


def attn_block(cfg, qkv, qn, kn, rtab, pos, kv):
    """attention_block after the qkv draw; kv (seq*row bytes, uint8) is updated in place."""
    assert kv.dtype == np.uint8 and kv.flags.c_contiguous
    if not 0 <= pos < cfg.seq or kv.size < cfg.seq * kv_row_bytes(cfg):
        raise ValueError("attn_block: pos %d outside the %d-row cache" % (pos, cfg.seq))
    out = np.empty(cfg.dim, np.int16)
    qn_ = None if qn is None else _c(qn, np.int16)
    kn_ = None if kn is None else _c(kn, np.int16)
    lib.vgxo_attn_block(ctypes.byref(cfg), _c(qkv, np.int16), _ptr(qn_), _ptr(kn_), _c(rtab, np.int32), pos,
                        kv, out)
    return out


def attn_parts(cfg, qrot, kv, pos):
    """(scores [heads, seq] int16, stats [heads, 2] int16, out [dim] int16)."""
    sc = np.zeros((cfg.heads, cfg.seq), np.int16)
    lib.vgxo_attn_scores(ctypes.byref(cfg), _c(qrot, np.int16), kv, pos, sc)
    st = np.empty((cfg.heads, 2), np.int16)
    lib.vgxo_attn_stats(ctypes.byref(cfg), sc, pos, st)
    out = np.empty(cfg.dim, np.int16)
    lib.vgxo_attn_v(ctypes.byref(cfg), sc, st, kv, pos, out)
    return sc, st, out


# ---- embedding / argmax / float path ------------------------------------------------
def conv_taps(w):
    """q16 taps [k][dim] of an f32 depthwise kernel w [dim][k]."""
    w = _c(w, np.float32)
    dim, k = w.shape
    out = np.empty((k, dim), np.int16)
    lib.vgxo_conv_taps(w, dim, k, out)
    return out


def conv_step(bcx, taps, state):
    """One position of the conv block: bcx [3*dim] q16, taps [3][dim] q16,
    state [2][dim] q16 (gated values of pos-2, pos-1; updated in place).
    Returns y [dim] q16."""
    dim = taps.shape[1]
    if state.dtype != np.int16 or not state.flags["C_CONTIGUOUS"] or state.shape != (2, dim):
        raise ValueError("state must be a contiguous int16 [2][dim] array")
    y = np.empty(dim, np.int16)
    s2, s1 = state[0], state[1]
    lib.vgxo_conv_step(dim, _c(bcx, np.int16), _c(taps, np.int16), s2, s1, y)
    return y


def embed_q8(emb, emb_scale, token):
    emb = _c(emb, np.int8)
    out = np.empty(emb.shape[1], np.int16)
    lib.vgxo_embed_q8(emb, _c(emb_scale, np.float32), emb.shape[1], int(token), out)
    return out


def argmax_i16(v):
    v = _c(v, np.int16)
    return int(lib.vgxo_argmax_i16(v, v.size))


def matvec_f32(w, x):
    w = _c(w, np.float32)
    out = np.empty(w.shape[0], np.float32)
    lib.vgxo_matvec_f32(w, w.shape[0], w.shape[1], _c(x, np.float32), out)
    return out


def rms_f32(x, w, eps):
    x = _c(x, np.float32)
    out = np.empty(x.size, np.float32)
    lib.vgxo_rms_f32(x, _ptr(None if w is None else _c(w, np.float32)), x.size, eps, out)
    return out


def threads():
    return int(lib.vgxo_threads())


def set_threads(n):
    lib.vgxo_set_threads(int(n))
