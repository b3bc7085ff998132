"""Whole-model oracle: the reference engine's decode step on the q16 grid, and
the reference's float CPU path, over an MMCF container.

TEST INFRASTRUCTURE ONLY (tests/, smoke, bench.py's cpu_baseline).  The
container is parsed here with its own small reader (the layout of
docs/checkpoint-container.md:62-271), independent of the product's.

QModel.step follows Session::forward_gpu_hidden (engine/src/session.cpp:1459-1584)
with the GPU kernels' numerics (oracle.py); FModel.step follows
engine/tools/ref_forward.py:47-115 on the dequantised container weights (CFModel
runs the same forward through the C/OpenMP float path, oracle/vgx_float.c), with
the engine's conventions (block RMSNorm eps from key 11 or 1e-5, q/k RMSNorm
eps 1e-6, RoPE tables of Session, engine/src/session.cpp:188-202).  With the
reference tools' conventions (qk_eps=None, tied_head=True) FModel reproduces
engine/tools/ref_generate.py, ref_forward.py and mmcf_hf.py
residual_peaks_lfm2 within fp32 summation order on vectors those tools wrote
(tests/test_float_pin.py, tests/golden/make_float_vectors.py).
"""
import ctypes
import os
import struct

import numpy as np

import oracle as o


def parse(blob):
    """(meta dict, {id: (dtype, rows, cols, scale, body ndarray uint8)})."""
    b = memoryview(blob)
    assert bytes(b[:4]) == b"MMCF"
    ver, hsz, n, _caps, moff, msize, doff, _fsize = struct.unpack_from("<HHIIIIQQ", b, 4)
    assert ver == 2 and hsz == 64
    meta, p = {}, moff
    while p + 8 <= moff + msize:
        key, _t, ln = struct.unpack_from("<HHI", b, p)
        meta[key] = bytes(b[p + 8:p + 8 + ln])
        p += 8 + ln
    recs = {}
    table = doff - 48 * n
    for i in range(n):
        r = table + 48 * i
        tid, dt, _fl, _g, _pad = struct.unpack_from("<HBBBB", b, r)
        rows, cols, off, nb = struct.unpack_from("<IIQQ", b, r + 6)
        scale, = struct.unpack_from("<f", b, r + 34)
        recs[tid] = (dt, rows, cols, scale, np.frombuffer(b[doff + off:doff + off + nb], np.uint8))
    return meta, recs


class _Mat:
    def __init__(self, kind, rows, cols, body, scale, prebiased=1, plane=None, s16=None, m16=None, mul=1.0):
        self.kind, self.rows, self.cols, self.body, self.scale = kind, rows, cols, body, scale
        self.prebiased, self.plane, self.s16, self.m16, self.mul = prebiased, plane, s16, m16, mul

    def wsr(self):
        s = np.float32(self.scale) * (np.float32(127) if self.kind == "t3" else np.float32(1))
        return o.row_scales(self.rows, float(np.float32(s) * np.float32(self.mul)), self.plane)

    def cols_slice(self, a, b):
        if self.kind == "q8":
            body = np.ascontiguousarray(self.body.reshape(self.rows, self.cols)[:, a:b])
            return _Mat("q8", self.rows, b - a, body, self.scale, self.prebiased, self.plane, mul=self.mul)
        if self.kind == "q4":
            g = self.cols // 32
            body = np.ascontiguousarray(self.body.reshape(self.rows, self.cols // 2)[:, a // 2:b // 2])
            s16 = np.ascontiguousarray(self.s16.reshape(self.rows, g)[:, a // 32:b // 32])
            m16 = np.ascontiguousarray(self.m16.reshape(self.rows, g)[:, a // 32:b // 32])
            return _Mat("q4", self.rows, b - a, body, self.scale, s16=s16, m16=m16, mul=self.mul)
        body = np.ascontiguousarray(self.body.reshape((self.rows + 1) // 2, self.cols // 8, 4)[:, a // 8:b // 8])
        return _Mat("t3", self.rows, b - a, body, self.scale, plane=self.plane, mul=self.mul)

    def rowval(self, x):
        if self.kind == "q8":
            return o.rowval_q8(self.body, self.prebiased, self.rows, self.cols, self.wsr(), x)
        if self.kind == "q4":
            ps = float(np.float32(self.scale) * np.float32(self.mul))
            return o.rowval_q4(self.body, self.s16, self.m16, ps, self.rows, self.cols, x)
        return o.rowval_t3(self.body, self.rows, self.cols, self.wsr(), x)

    def dequant(self):
        if self.kind == "q8":
            return o.dequant_q8(self.body, self.prebiased, self.rows, self.cols, self.wsr())
        if self.kind == "q4":
            ps = float(np.float32(self.scale) * np.float32(self.mul))
            return o.dequant_q4(self.body, self.s16, self.m16, ps, self.rows, self.cols)
        return o.dequant_t3(self.body, self.rows, self.cols, self.wsr())


class _Base:
    def __init__(self, blob, seq=None, kv_bits=16):
        meta, self.recs = parse(blob)
        d = struct.unpack("<7i", meta[1])
        self.dim, self.hidden, self.layers, self.heads, self.kv_heads, self.vocab, seq0 = d
        self.seq = seq or seq0
        th, half, qk, _ = struct.unpack("<fBBH", meta[2])
        self.theta, self.rope_half, self.qk_norm = th, half, qk
        self.eps = struct.unpack("<f", meta[11])[0] if 11 in meta else 1e-5
        self.hid = list(meta.get(15, b"")) or [0] * self.layers
        self.hd = self.dim // self.heads
        self.kv_dim = self.kv_heads * self.hd
        self.kv_bits = kv_bits
        self.chunk = (self.hidden + 1) // 2 if self.hidden > 2048 else 0
        # key 14: nonzero = an LFM2 conv layer (in_proj 0x17, f32 depthwise
        # kernel 0x18, out_proj 0x19; engine/src/model.cpp:1142-1160)
        self.is_conv = list(meta.get(14, b"")) or [0] * self.layers
        self.conv_w = [None] * self.layers
        self.mats = []
        for l in range(self.layers):
            if self.is_conv[l]:
                L = {"conv_in": self.mat(0x17, l), "conv_out": self.mat(0x19, l)}
                _dt, rows, cols, _s, body = self.recs[0x18 | l << 8]
                self.conv_w[l] = body.view(np.float32).reshape(rows, cols)
            else:
                L = {"qkv": self.mat(0x10, l), "wo": self.mat(0x11, l)}
            if (0x14 | l << 8) in self.recs:
                w13 = self.mat(0x14, l)
                L["w1"], L["w3"] = self.rows_of(w13, 0, self.hidden), self.rows_of(w13, self.hidden, 2 * self.hidden)
            else:
                L["w1"], L["w3"] = self.mat(0x12, l), self.mat(0x13, l)
            L["w2"] = self.mat(0x15, l, mul=float(1 << self.hid[l]))
            self.mats.append(L)
        self.emb = self.recs[1][4].view(np.int8).reshape(self.vocab, self.dim)
        self.es = self.recs[2][4].view(np.float32)
        self.tiles = []
        i = 0
        while (0x20 | i << 8) in self.recs:
            self.tiles.append(self.mat(0x20, i))
            i += 1
        if not self.tiles:
            unit = self.es.max()
            for st in range(0, self.vocab, 1536):
                rows = min(1536, self.vocab - st)
                body = np.ascontiguousarray(self.emb[st:st + rows]).view(np.uint8)
                self.tiles.append(_Mat("q8", rows, self.dim, body, float(unit), 0,
                                       (self.es[st:st + rows] / np.float32(unit)).astype(np.float32)))
        f32 = lambda k: self.recs[k][4].view(np.float32)
        self.rms_att = f32(3).reshape(self.layers, self.dim)
        self.rms_ffn = f32(4).reshape(self.layers, self.dim)
        self.rms_final = f32(5)
        self.qn = f32(6).reshape(self.layers, self.hd) if self.qk_norm else None
        self.kn = f32(7).reshape(self.layers, self.hd) if self.qk_norm else None
        self.rcos, self.rsin = o.rope_cos_sin(self.theta, self.hd, self.seq)

    def mat(self, kind, layer, mul=1.0):
        base = kind | (layer << 8)
        dt, rows, cols, scale, body = self.recs[base]
        plane = self.recs[base | (3 << 14)][4].view(np.float32) if (base | (3 << 14)) in self.recs else None
        if dt in (2, 3):
            return _Mat("q8", rows, cols, body, scale, 1 if dt == 2 else 0, plane, mul=mul)
        if dt == 7:
            return _Mat("t3", rows, cols, body, scale, plane=plane, mul=mul)
        if dt == 4:
            return _Mat("q4", rows, cols, body, scale, s16=self.recs[base | (1 << 14)][4].view(np.int16),
                        m16=self.recs[base | (2 << 14)][4].view(np.int16), mul=mul)
        raise ValueError("dtype %d" % dt)

    @staticmethod
    def rows_of(m, a, b):
        if m.kind == "q8":
            return _Mat("q8", b - a, m.cols, m.body.reshape(m.rows, m.cols)[a:b].ravel(), m.scale, m.prebiased,
                        None if m.plane is None else m.plane[a:b], mul=m.mul)
        if m.kind == "q4":
            g = m.cols // 32
            return _Mat("q4", b - a, m.cols, m.body.reshape(m.rows, m.cols // 2)[a:b].ravel(), m.scale,
                        s16=m.s16.reshape(m.rows, g)[a:b].ravel(), m16=m.m16.reshape(m.rows, g)[a:b].ravel(),
                        mul=m.mul)
        st = (m.cols // 8) * 4
        return _Mat("t3", b - a, m.cols, m.body[(a // 2) * st:((b + 1) // 2) * st], m.scale,
                    plane=m.plane[a:b], mul=m.mul)


class QModel(_Base):
    """The engine's decode step on the q16 grid; logits are q16 integers."""

    def __init__(self, blob, seq=None, kv_bits=16):
        super().__init__(blob, seq, kv_bits)
        self.cfg = o.attn_cfg(self.dim, self.heads, self.kv_heads, self.hd, self.seq, kv_bits,
                              self.rope_half, self.qk_norm)
        self.rtab = o.rope_table(self.rcos, self.rsin)
        self.kv = [np.zeros(self.seq * o.kv_row_bytes(self.cfg), np.uint8) for _ in range(self.layers)]
        self.w_att = [o.quantize_act(self.rms_att[l]) for l in range(self.layers)]
        self.w_ffn = [o.quantize_act(self.rms_ffn[l]) for l in range(self.layers)]
        self.w_fin = o.quantize_act(self.rms_final)
        self.qnq = [o.quantize_act(self.qn[l]) for l in range(self.layers)] if self.qk_norm else None
        self.knq = [o.quantize_act(self.kn[l]) for l in range(self.layers)] if self.qk_norm else None
        if self.chunk:
            self.w2ab = [(L["w2"].cols_slice(0, self.chunk), L["w2"].cols_slice(self.chunk, self.hidden))
                         for L in self.mats]
        self.taps = [o.conv_taps(w) if w is not None else None for w in self.conv_w]
        self.conv_state = [np.zeros((2, self.dim), np.int16) for _ in range(self.layers)]

    def step(self, token, pos, want_logits=True):
        if pos == 0:  # a new sequence starts with an empty conv history
            for st in self.conv_state:
                st[:] = 0
        h = o.embed_q8(self.emb, self.es, token)
        for l, L in enumerate(self.mats):
            xb = o.rmsnorm(h, self.w_att[l], self.eps)
            if self.is_conv[l]:
                # GPU::conv_block (engine/src/gpu_conv.cpp:165-225)
                bcx = o.store(L["conv_in"].rowval(xb))
                y = o.conv_step(bcx, self.taps[l], self.conv_state[l])
                x1 = o.store(L["conv_out"].rowval(y), h)
            else:
                qkv = o.store(L["qkv"].rowval(xb))
                att = o.attn_block(self.cfg, qkv, self.qnq[l] if self.qnq else None,
                                   self.knq[l] if self.knq else None, self.rtab, pos, self.kv[l])
                x1 = o.store(L["wo"].rowval(att), h)
            xb = o.rmsnorm(x1, self.w_ffn[l], self.eps)
            hb = o.gate(L["w1"].rowval(xb), L["w3"].rowval(xb), self.hid[l])
            if self.chunk:
                a, b = self.w2ab[l]
                h = o.store(b.rowval(hb[self.chunk:]), o.store(a.rowval(hb[:self.chunk]), x1))
            else:
                h = o.store(L["w2"].rowval(hb), x1)
        if not want_logits:
            return None
        xf = o.rmsnorm(h, self.w_fin, self.eps)
        return np.concatenate([o.store(t.rowval(xf)) for t in self.tiles])


def rowval_q4_view4(nib, s16, m16, ps, rows, cols, x):
    """Row values of a q4 matrix as the reference's 4-bit texture view
    evaluates them, step by step in IEEE fp32 with round-to-nearest and no
    fused multiply-add: matvec_i4_add_4x4 (engine/src/shaders.cpp:1754-1782);
    the gate's i4_gate_flat8b (shaders.cpp:1539-1590) and the qkv's
    matvec_i4_4x4 accumulate the same way.

    The view differs from the packed form only in rounding:
    - a weight nibble n is sampled from GL_RGBA4 as UNORM, fp32(n/15);
    - the group scale is unsigned, sampled as two UNORM8 bytes
      (engine/src/gpu_upload.cpp:170-180: r = s16 >> 8, g = s16 & 255) and
      rebuilt as r*(65280*15*ps) + g*(255*15*ps);
    - the group minimum goes through x_i16raw (r*65280 + g*255, minus 65536
      at or above 32767.5) times ps;
    - per 8 columns, d += w0.x*xa.x + ... + w1.w*xb.w left to right;
    - per group, s += sc*d + mn*xsum.
    What the driver does with the UNORM conversions and whether its compiler
    fuses multiply-adds is not in the reference's sources, so this is a model
    of one conforming evaluation, not of a measured device."""
    f = np.float32
    ps = f(ps)
    G = cols // 32
    b = np.asarray(nib, np.uint8).reshape(rows, cols // 2)
    n = np.empty((rows, cols), np.uint8)
    n[:, 0::2], n[:, 1::2] = b & 15, b >> 4
    w = n.astype(f) / f(15)
    xf = np.asarray(x, np.int16).astype(f)
    u, v = f(f(979200) * ps), f(f(3825) * ps)
    su = np.asarray(s16, np.int16).reshape(rows, G).view(np.uint16)
    sc = (su >> 8).astype(f) / f(255) * u + (su & 255).astype(f) / f(255) * v
    mu = np.asarray(m16, np.int16).reshape(rows, G).view(np.uint16)
    raw = (mu >> 8).astype(f) / f(255) * f(65280) + (mu & 255).astype(f) / f(255) * f(255)
    mn = np.where(raw >= f(32767.5), raw - f(65536), raw).astype(f) * ps
    p = (w * xf).reshape(rows, G, 4, 8)
    e = p[..., 0]
    for j in range(1, 8):
        e = e + p[..., j]
    d = e[..., 0]
    for t in range(1, 4):
        d = d + e[..., t]
    # xsum is a sum of at most 32 integers of 16 bits: exact in fp32
    xsum = xf.reshape(G, 32).astype(np.int64).sum(axis=1).astype(f)
    term = sc * d + mn * xsum
    s = term[:, 0]
    for g in range(1, G):
        s = s + term[:, g]
    return s.astype(f)


class _Mat4(_Mat):
    """A q4 matrix read through the 4-bit texture view."""

    def rowval(self, x):
        ps = float(np.float32(self.scale) * np.float32(self.mul))
        return rowval_q4_view4(self.body, self.s16, self.m16, ps, self.rows, self.cols, x)

    @staticmethod
    def of(m):
        if m.kind != "q4":
            return m
        return _Mat4(m.kind, m.rows, m.cols, m.body, m.scale, m.prebiased, m.plane, m.s16, m.m16, m.mul)


class QModelView4(QModel):
    """QModel with the reference's default q4 path: Model::apply_q4_fmt
    (engine/src/model.cpp:337-400) marks every q4 qkv, wo, gate, w2 chunk and
    conv projection of a chunked-FFN model (hidden > 2048) for the 4-bit view
    unless Q4_FMT=0; an unchunked model keeps the packed view, as QModel."""

    def __init__(self, blob, seq=None, kv_bits=16):
        super().__init__(blob, seq, kv_bits)
        if not self.chunk:
            return
        self.mats = [{k: _Mat4.of(m) for k, m in L.items()} for L in self.mats]
        self.w2ab = [(_Mat4.of(a), _Mat4.of(b)) for a, b in self.w2ab]


class FModel(_Base):
    """The float CPU path on the dequantised container weights.

    qk_eps: the q/k RMSNorm eps.  The engine uses 1e-6
    (engine/src/shaders_attn.cpp:259-268); the reference's float tools use the
    block eps for both (engine/tools/ref_forward.py:75-78,
    engine/tools/ref_generate.py:88-90), which qk_eps=None selects.
    tied_head: the LM head is the float embedding itself (emb * es), as those
    tools compute logits (`x @ emb.T`, ref_forward.py:113); the default is the
    container's q8 head tiles, which is what the engine multiplies by."""

    def __init__(self, blob, seq=None, qk_eps=1e-6, tied_head=False):
        super().__init__(blob, seq)
        self.qk_eps = self.eps if qk_eps is None else qk_eps
        # key 15's 2^k on w2 only undoes the hidden's q16 store scale, which
        # the float path does not apply
        self.W = []
        for L in self.mats:
            w2 = L["w2"]
            L = dict(L, w2=_Mat(w2.kind, w2.rows, w2.cols, w2.body, w2.scale, w2.prebiased, w2.plane,
                                w2.s16, w2.m16, 1.0))
            self.W.append({k: m.dequant() for k, m in L.items()})
        if tied_head:
            self.head = self.emb.astype(np.float32) * self.es[:, None]
        else:
            self.head = np.concatenate([t.dequant() for t in self.tiles])
        self.kc = np.zeros((self.layers, self.seq, self.kv_heads, self.hd), np.float32)
        self.vc = np.zeros_like(self.kc)
        self.cstate = np.zeros((self.layers, 2, self.dim), np.float32)  # B*x of pos-2, pos-1

    def _rope(self, x, pos):
        c, s = self.rcos[pos], self.rsin[pos]
        if self.rope_half:
            x1, x2 = x[..., :self.hd // 2], x[..., self.hd // 2:]
            return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)
        out = np.empty_like(x)
        out[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
        out[..., 1::2] = x[..., 1::2] * c + x[..., 0::2] * s
        return out

    def _per_q_head(self, kv):
        """[t, kv_heads, hd] -> [t, heads, hd]: query head h reads KV head
        h // (heads / kv_heads) (GQA, ref_forward.py:85-86)."""
        return np.repeat(kv, self.heads // self.kv_heads, axis=1)

    @staticmethod
    def _rms(x, w, eps):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w

    def _conv(self, l, W, xn):
        """LFM2 ShortConv in float: B, C, x = in_proj(xn); Bx = B*x; a causal
        depthwise conv over the last three Bx (tap 0 on pos-2); C * conv;
        out_proj (the CPU form of Session, engine/src/session.cpp:383-418,
        without its q16 stores)."""
        bcx = W["conv_in"] @ xn
        b, c, xx = bcx[:self.dim], bcx[self.dim:2 * self.dim], bcx[2 * self.dim:]
        bx = b * xx
        w = self.conv_w[l]
        st = self.cstate[l]
        cv = w[:, 0] * st[0] + w[:, 1] * st[1] + w[:, 2] * bx
        st[0], st[1] = st[1], bx
        return W["conv_out"] @ (c * cv)

    def step(self, token, pos, trace=None):
        """Logits of position pos; trace (a list, optional) receives the
        residual after each layer."""
        if pos == 0:
            self.cstate[:] = 0
        x = self.emb[token].astype(np.float32) * self.es[token]
        for l, W in enumerate(self.W):
            xn = self._rms(x, self.rms_att[l], self.eps)
            if self.is_conv[l]:
                x = x + self._conv(l, W, xn)
                xn = self._rms(x, self.rms_ffn[l], self.eps)
                g, u = W["w1"] @ xn, W["w3"] @ xn
                x = x + W["w2"] @ ((g / (1 + np.exp(-g))) * u)
                if trace is not None:
                    trace.append(x.copy())
                continue
            qkv = W["qkv"] @ xn
            q = qkv[:self.dim].reshape(self.heads, self.hd)
            k = qkv[self.dim:self.dim + self.kv_dim].reshape(self.kv_heads, self.hd)
            v = qkv[self.dim + self.kv_dim:].reshape(self.kv_heads, self.hd)
            if self.qk_norm:
                q = self._rms(q, self.qn[l], self.qk_eps)
                k = self._rms(k, self.kn[l], self.qk_eps)
            q, k = self._rope(q, pos), self._rope(k, pos)
            self.kc[l, pos], self.vc[l, pos] = k, v
            K, V = self._per_q_head(self.kc[l, :pos + 1]), self._per_q_head(self.vc[l, :pos + 1])
            sc = np.einsum("hd,thd->ht", q, K) / np.sqrt(self.hd)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            att = np.einsum("ht,thd->hd", p, V).reshape(self.dim)
            x = x + W["wo"] @ att
            xn = self._rms(x, self.rms_ffn[l], self.eps)
            g, u = W["w1"] @ xn, W["w3"] @ xn
            x = x + W["w2"] @ ((g / (1 + np.exp(-g))) * u)
            if trace is not None:
                trace.append(x.copy())
        return self.head @ self._rms(x, self.rms_final, self.eps)


class _VgxfModel(ctypes.Structure):
    _P = ctypes.c_void_p
    _fields_ = [(n, ctypes.c_int) for n in ("dim", "hidden", "layers", "heads", "kv_heads", "head_dim", "vocab",
                                            "seq", "rope_half", "qk_norm")] + \
               [("eps", ctypes.c_float)] + \
               [(n, ctypes.c_void_p) for n in ("is_conv", "qkv", "wo", "conv_in", "conv_out", "conv_w", "w1", "w3",
                                               "w2", "rms_att", "rms_ffn", "rms_final", "qn", "kn", "rcos", "rsin",
                                               "emb", "es", "head")]


_FLIB = None


def float_lib():
    """oracle/lib/libvgx_float.so: the float path in C (oracle/vgx_float.c)."""
    global _FLIB
    if _FLIB is None:
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libvgx_float.so")
        if not os.path.exists(path):
            raise RuntimeError("float-path library missing: run `make -C oracle` (%s)" % path)
        L = ctypes.CDLL(path)
        L.vgxf_state_new.restype = ctypes.c_void_p
        L.vgxf_state_new.argtypes = [ctypes.c_void_p]
        L.vgxf_state_free.argtypes = [ctypes.c_void_p]
        L.vgxf_step.restype = ctypes.c_int
        L.vgxf_step.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        L.vgxf_threads.restype = ctypes.c_int
        L.vgxf_set_threads.argtypes = [ctypes.c_int]
        _FLIB = L
    return _FLIB


class CFModel(FModel):
    """FModel's float forward run by the C/OpenMP float path (oracle/vgx_float.c)
    on the same dequantised arrays: the CPU baseline of the decode benchmarks."""

    def __init__(self, blob, seq=None):
        super().__init__(blob, seq)
        keep = []

        def arr(a, dt=np.float32):
            a = np.ascontiguousarray(a, dtype=dt)
            keep.append(a)
            return a.ctypes.data

        def ptrs(key):
            p = (ctypes.c_void_p * self.layers)(*[arr(W[key]) if key in W else None for W in self.W])
            keep.append(p)
            return ctypes.cast(p, ctypes.c_void_p)

        cw = (ctypes.c_void_p * self.layers)(*[arr(w) if w is not None else None for w in self.conv_w])
        keep.append(cw)
        m = _VgxfModel(dim=self.dim, hidden=self.hidden, layers=self.layers, heads=self.heads,
                       kv_heads=self.kv_heads, head_dim=self.hd, vocab=self.vocab, seq=self.seq,
                       rope_half=int(bool(self.rope_half)), qk_norm=int(bool(self.qk_norm)), eps=self.eps)
        m.is_conv = arr(np.array(self.is_conv, np.int32), np.int32)
        for key in ("qkv", "wo", "conv_in", "conv_out", "w1", "w3", "w2"):
            setattr(m, key, ptrs(key))
        m.conv_w = ctypes.cast(cw, ctypes.c_void_p)
        m.rms_att, m.rms_ffn, m.rms_final = arr(self.rms_att), arr(self.rms_ffn), arr(self.rms_final)
        if self.qk_norm:
            m.qn, m.kn = arr(self.qn), arr(self.kn)
        m.rcos, m.rsin = arr(self.rcos), arr(self.rsin)
        m.emb, m.es, m.head = arr(self.emb, np.int8), arr(self.es), arr(self.head)
        self._keep, self._m = keep, m
        self._st = float_lib().vgxf_state_new(ctypes.byref(m))
        if not self._st:
            raise MemoryError("vgxf_state_new")

    def step(self, token, pos, logits=True):
        out = np.empty(self.vocab, np.float32) if logits else None
        rc = float_lib().vgxf_step(ctypes.byref(self._m), self._st, int(token), int(pos),
                                   out.ctypes.data if logits else None)
        if rc:
            raise ValueError("vgxf_step: token or position out of range")
        return out

    def __del__(self):
        if getattr(self, "_st", None):
            float_lib().vgxf_state_free(self._st)
            self._st = None
