"""MMCF v2 containers: quantizers, writer and reader.

The byte contract the decode kernels consume.  The layout follows
docs/checkpoint-container.md:62-271 of the reference (header, TLV metadata,
48-byte tensor records, 16-byte aligned bodies, q8 stored XOR 0x80 as q8u8);
the quantizers follow engine/tools/mmcf_hf.py with numpy float32 arithmetic
(a Python float meeting a float32 array is cast to float32 first, NEP 50) and
round-half-even, so a container written here is byte-identical to the
reference packer's for the same float weights.
"""
import math
import struct
import zlib
from dataclasses import dataclass, field

import numpy as np

MAGIC = b"MMCF"
HEADER_SIZE = 64
REC_SIZE_V2 = 48
ALIGN = 16
LOGITS_GRID = 1536  # engine/src/logits_grid.h:38

# dtypes (docs/checkpoint-container.md "Dtypes")
DT_F32, DT_I16, DT_Q8U8, DT_Q8I8, DT_Q4, DT_BLOB, DT_Q6, DT_T3 = range(8)
# tensor kinds; id = kind | layer << 8 | part << 14
T_EMB, T_EMB_SCALE, T_RMS_ATT, T_RMS_FFN, T_RMS_FINAL, T_Q_NORM, T_K_NORM = 1, 2, 3, 4, 5, 6, 7
T_QKV, T_WO, T_W1, T_W3, T_W13, T_W2 = 0x10, 0x11, 0x12, 0x13, 0x14, 0x15
T_CONV_IN, T_CONV_W, T_CONV_OUT = 0x17, 0x18, 0x19
T_LOGITS = 0x20
SCHEMES = {"i16": 0, "q8": 1, "q4": 2, "t3": 3}


# ---------------------------------------------------------------------------
# quantizers (engine/tools/mmcf_hf.py)

def qmat(w):
    """Per-matrix int16: s = max|w|/32767 (a Python float), q = rint(w/s)."""
    w = np.asarray(w, np.float32)
    mx = float(np.abs(w).max()) if w.size else 0.0
    s = (mx if mx != 0 else 1.0) / 32767.0
    q = np.clip(np.rint(w / np.float32(s)), -32767, 32767).astype(np.int16)
    return q, s


def q8mat(w):
    """Per-matrix int8 at s = max|w|/127 (mmcf_hf.py:60-66)."""
    w = np.asarray(w, np.float32)
    mx = float(np.abs(w).max()) if w.size else 0.0
    s = (mx if mx != 0 else 1.0) / 127.0
    q = np.clip(np.rint(w / np.float32(s)), -127, 127).astype(np.int8)
    return q, s


def q8_from_i16(w):
    """The two-step q8 of a q8 container: int16 first, dequantised, then q8."""
    q, s = qmat(w)
    return q8mat(q.astype(np.float32) * np.float32(s))


def q8_per_row(w):
    """One scale per output row: (q, unit = max row scale, plane = s_row/unit)."""
    w = np.asarray(w, np.float32)
    s = np.abs(w).max(axis=1, keepdims=True) / np.float32(127.0)
    s[s == 0] = 1.0
    q = np.clip(np.rint(w / s), -127, 127).astype(np.int8)
    unit = float(s.max())
    return q, unit, (s[:, 0] / np.float32(unit)).astype(np.float32)


def q4mat(w):
    """Groups of 32, asymmetric: nibbles (even column in the low nibble), int16
    scale and min planes at one shared step ps (mmcf_hf.py:69-91)."""
    w = np.asarray(w, np.float32)
    rows, cols = w.shape
    if cols % 32:
        raise ValueError("q4 cols must be divisible by 32: %dx%d" % (rows, cols))
    groups = cols // 32
    z = w.reshape(rows, groups, 32)
    lo = z.min(axis=2, keepdims=True)
    hi = z.max(axis=2, keepdims=True)
    sc = (hi - lo) / np.float32(15.0)
    sc[sc == 0] = 1.0
    q = np.clip(np.rint((z - lo) / sc), 0, 15).astype(np.uint8).reshape(rows, cols)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    flat_sc, flat_lo = sc[:, :, 0], lo[:, :, 0]
    m = max(np.abs(flat_sc).max(), np.abs(flat_lo).max())
    if float(m) > 1e-12:
        ps = float(np.float32(m) / np.float32(32767.0))
    else:
        ps = 1e-12 / 32767.0
    s16 = np.clip(np.rint(flat_sc / np.float32(ps)), -32767, 32767).astype("<i2")
    m16 = np.clip(np.rint(flat_lo / np.float32(ps)), -32767, 32767).astype("<i2")
    return packed, s16, m16, ps, groups


def _t3_byte_index(rows, cols):
    """Byte of weight (r, c) in the texel grid and its bit shift, from the
    container's texel formula (docs/checkpoint-container.md, "t3"): texel
    (c8, t) is 4 bytes at t*stride + 4*c8; row 2t's columns 8c8..8c8+3 are
    byte 0, 8c8+4..8c8+7 byte 1, row 2t+1 the same in bytes 2 and 3; weight k
    of a byte sits at bits 2k."""
    stride = (cols // 8) * 4
    r = np.arange(rows)[:, None]
    c = np.arange(cols)[None, :]
    byte = (r // 2) * stride + (c // 8) * 4 + (r % 2) * 2 + (c // 4) % 2
    return byte, 2 * (c % 4)


def t3_codes_pack(code):
    """(rows, cols) 2-bit codes, rows even and cols a multiple of 8 -> the texel
    grid bytes, (rows/2, cols/2) per texel row."""
    rows, cols = code.shape
    byte, shift = _t3_byte_index(rows, cols)
    out = np.zeros((rows // 2) * (cols // 8) * 4, np.uint8)
    for k in range(4):  # each byte holds one weight of each column phase k
        out[byte[:, k::4].ravel()] |= ((code[:, k::4].astype(np.uint8) & 3) << (2 * k)).ravel()
    return out.reshape(rows // 2, -1)


def t3_codes_unpack(block, rows, cols):
    rpad, cpad = rows + (rows % 2), cols + ((-cols) % 8)
    body = np.frombuffer(bytes(block), np.uint8)
    byte, shift = _t3_byte_index(rpad, cpad)
    return ((body[byte] >> shift) & 3).astype(np.uint8)[:rows, :cols]


def t3_levels(codes):
    """bit 0 magnitude, bit 1 sign: level = mag * (1 - 2*sign)."""
    c = codes.astype(np.int8)
    return (c & 1) * (1 - 2 * ((c >> 1) & 1))


def t3mat(w):
    """A per-row ternary matrix -> (2-bit texel bytes, unit, plane), certified
    as mmcf_hf.t3mat does (row_ternary at rtol 1e-3, exact decode)."""
    w = np.asarray(w, np.float32)
    rows, cols = w.shape
    a = np.abs(w)
    mx = a.max(axis=1, keepdims=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        rel = np.abs(a - mx) / np.maximum(mx, np.float32(1e-30))
    if not ((a == 0) | (rel <= 1e-3)).all():
        raise ValueError("t3mat: matrix is not per-row ternary")
    s = a.max(axis=1) / np.float32(127.0)
    s[s == 0] = 1.0
    lev = np.rint(w / (s[:, None] * np.float32(127.0)))
    code = (np.abs(lev) > 0.5).astype(np.uint8) | ((lev < -0.5).astype(np.uint8) << 1)
    pad = (-cols) % 8
    if pad:
        code = np.pad(code, ((0, 0), (0, pad)))
    if rows % 2:
        code = np.pad(code, ((0, 1), (0, 0)))
    packed = t3_codes_pack(code).tobytes()
    unit = float(s.max())
    back = t3_levels(t3_codes_unpack(packed, rows, cols)).astype(np.float32) * (s[:, None] * np.float32(127.0))
    if w.size and float(np.abs(back - w).max()) > 1e-6 * max(1.0, float(a.max())):
        raise ValueError("t3mat: pack/unpack is not exact")
    return packed, unit, (s / np.float32(unit)).astype(np.float32)


# ---------------------------------------------------------------------------
# container writer

def _tlv(key, payload):
    return struct.pack("<HHI", key, 1, len(payload)) + payload


def _rec(tid, dt, group, rows, cols, off, blen, crc, scale):
    b = struct.pack("<HBBBB", tid, dt, 0, group, 0) + struct.pack("<II", rows, cols)
    b += struct.pack("<QQ", off, blen) + struct.pack("<I", crc) + struct.pack("<f", float(scale))
    b += struct.pack("<H", 0)
    return b + b"\0" * (REC_SIZE_V2 - len(b))


@dataclass
class ModelSpec:
    """A dense decoder in the shape the container describes (metadata key 1/2)."""
    dim: int
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    vocab: int
    seq: int
    theta: float = 10000.0
    rope_half: bool = True
    qk_norm: bool = False
    layer_types: list = field(default_factory=list)  # 'attn' / 'conv' (key 14)
    hid_scale: list = field(default_factory=list)    # key 15
    rms_eps: float = None                            # key 11

    @property
    def head_dim(self):
        return self.dim // self.heads

    @property
    def kv_dim(self):
        return self.kv_heads * self.head_dim


def tensors_from_float(spec, w, scheme, q8_row=False, head_dedup=False):
    """The tensor list (id, dtype, rows, cols, group, payload, scale) a float
    model packs to, in the order mmcf_hf.tensors_from_hf writes it
    (mmcf_hf.py:1783-2011).  `w` holds float32 arrays: emb [vocab,dim],
    rms_att/rms_ffn [layers,dim], rms_final [dim], q_norm/k_norm [layers,hd]
    (qk_norm), wq/wk/wv/wo/w1/w3/w2 per layer, wcls [vocab,dim] (tied: emb)."""
    T = []
    L = spec.layers

    def f32(a):
        return np.asarray(a, np.float32).tobytes()

    er = np.empty((spec.vocab, spec.dim), np.int8)
    es = np.empty(spec.vocab, np.float32)
    for i in range(spec.vocab):
        row = np.asarray(w["emb"][i], np.float32)
        er[i], s = q8_from_i16(row) if scheme == "q8" else q8mat(row)
        es[i] = s
    T.append((T_EMB, DT_Q8I8, spec.vocab, spec.dim, 0, er.tobytes(), 0.0))
    T.append((T_EMB_SCALE, DT_F32, spec.vocab, 1, 0, es.tobytes(), 0.0))
    T.append((T_RMS_ATT, DT_F32, L, spec.dim, 0, f32(w["rms_att"]), 0.0))
    T.append((T_RMS_FFN, DT_F32, L, spec.dim, 0, f32(w["rms_ffn"]), 0.0))
    T.append((T_RMS_FINAL, DT_F32, 1, spec.dim, 0, f32(w["rms_final"]), 0.0))
    if spec.qk_norm:
        T.append((T_Q_NORM, DT_F32, L, spec.head_dim, 0, f32(w["q_norm"]), 0.0))
        T.append((T_K_NORM, DT_F32, L, spec.head_dim, 0, f32(w["k_norm"]), 0.0))

    def mat(tid, layer, m):
        m = np.asarray(m, np.float32)
        rows, cols = m.shape
        base = tid | (layer << 8)
        if scheme == "q8" and q8_row:
            q, unit, plane = q8_per_row(m)
            T.append((base, DT_Q8I8, rows, cols, 0, q.tobytes(), unit))
            T.append((base | (3 << 14), DT_F32, rows, 1, 0, plane.astype("<f4").tobytes(), 0.0))
        elif scheme == "q8":
            q, s = q8_from_i16(m)
            T.append((base, DT_Q8I8, rows, cols, 0, q.tobytes(), s))
        elif scheme == "t3":
            packed, unit, plane = t3mat(m)
            T.append((base, DT_T3, rows, cols, 0, packed, unit))
            T.append((base | (3 << 14), DT_F32, rows, 1, 0, plane.astype("<f4").tobytes(), 0.0))
        elif scheme == "q4":
            packed, s16, m16, ps, groups = q4mat(m)
            T.append((base, DT_Q4, rows, cols, 32, packed.tobytes(), ps))
            T.append((base | (1 << 14), DT_I16, rows, groups, 0, s16.tobytes(), 0.0))
            T.append((base | (2 << 14), DT_I16, rows, groups, 0, m16.tobytes(), 0.0))
        else:
            raise ValueError("scheme %r" % scheme)

    split = 2 * spec.hidden > 2048
    types = spec.layer_types or ["attn"] * L
    for l in range(L):
        if types[l] == "conv":
            mat(T_CONV_IN, l, w["conv_in"][l])
            cw = np.asarray(w["conv_w"][l], np.float32)
            T.append((T_CONV_W | (l << 8), DT_F32, cw.shape[0], cw.shape[1], 0, cw.tobytes(), 0.0))
            mat(T_CONV_OUT, l, w["conv_out"][l])
        else:
            mat(T_QKV, l, np.concatenate([w["wq"][l], w["wk"][l], w["wv"][l]], axis=0))
            mat(T_WO, l, w["wo"][l])
        if split:
            mat(T_W1, l, w["w1"][l])
            mat(T_W3, l, w["w3"][l])
        else:
            mat(T_W13, l, np.concatenate([w["w1"][l], w["w3"][l]], axis=0))
        mat(T_W2, l, w["w2"][l])
    if head_dedup:
        # --head-dedup: a tied head is the embedding; no logits tiles are written
        return T
    wcls = w.get("wcls", w["emb"])
    for i, st in enumerate(range(0, spec.vocab, LOGITS_GRID)):
        tile = np.asarray(wcls[st:st + LOGITS_GRID], np.float32)
        if scheme != "q4":
            mat(T_LOGITS, i, tile)
        else:
            q, s = q8mat(tile)
            T.append((T_LOGITS | (i << 8), DT_Q8I8, tile.shape[0], tile.shape[1], 0, q.tobytes(), s))
    return T


def build(spec, tensors, scheme, name="model", template="chatml", system="You are a helpful assistant.",
          chat=False):
    """Container bytes (mmcf_pack.py:284-430): header, TLV metadata, tensor
    table, 16-byte aligned bodies; q8i8 bodies other than the embedding are
    stored XOR 0x80 as q8u8."""
    kinds = {"plain": 0, "qwen": 1, "chatml": 1, "minimind3": 2, "tinybrainbot": 3}
    md = _tlv(1, struct.pack("<7i", spec.dim, spec.hidden, spec.layers, spec.heads, spec.kv_heads,
                             spec.vocab, spec.seq))
    md += _tlv(2, struct.pack("<fBBH", float(spec.theta), 1 if spec.rope_half else 0,
                              1 if spec.qk_norm else 0, 0))
    md += _tlv(3, struct.pack("<BBBB", SCHEMES[scheme], 32 if scheme == "q4" else 0, 1,
                              1 if 2 * spec.hidden > 2048 else 0))
    md += _tlv(4, bytes([kinds[template]]) + system.encode() + b"\0" + template.encode() + b"\0")
    caps = 1 if chat else 0
    md += _tlv(5, struct.pack("<I", caps))
    md += _tlv(6, name.encode() + b"\0")
    if spec.rms_eps is not None:
        md += _tlv(11, struct.pack("<f", spec.rms_eps))
    if spec.layer_types:
        md += _tlv(14, bytes(1 if t == "conv" else 0 for t in spec.layer_types))
    if spec.hid_scale and any(spec.hid_scale):
        md += _tlv(15, bytes(int(k) for k in spec.hid_scale))
    table_off = HEADER_SIZE + len(md)
    table_off = (table_off + ALIGN - 1) // ALIGN * ALIGN
    data_off = table_off + len(tensors) * REC_SIZE_V2
    table, data = bytearray(), bytearray()
    for tid, dt, rows, cols, group, payload, scale in tensors:
        if dt == DT_Q8I8 and (tid & 0xFF) != T_EMB:
            payload = (np.frombuffer(payload, np.uint8) ^ 0x80).tobytes()
            dt = DT_Q8U8
        while (data_off + len(data)) % ALIGN:
            data.append(0)
        off = len(data)
        data += payload
        table += _rec(tid, dt, group, rows, cols, off, len(payload), zlib.crc32(payload) & 0xFFFFFFFF, scale)
    size = data_off + len(data)
    body = MAGIC + struct.pack("<HHIIIIQQ", 2, HEADER_SIZE, len(tensors), caps, HEADER_SIZE, len(md),
                               data_off, size)
    head = (body + struct.pack("<I", zlib.crc32(body) & 0xFFFFFFFF)).ljust(HEADER_SIZE, b"\0")
    out = bytearray(head) + md
    out += b"\0" * (table_off - len(out))
    return bytes(out + table + data)


# ---------------------------------------------------------------------------
# container reader (engine/src/model.cpp:873-1304 semantics)

@dataclass
class Record:
    tid: int
    dtype: int
    group: int
    rows: int
    cols: int
    scale: float
    body: memoryview

    @property
    def kind(self):
        return self.tid & 0xFF

    @property
    def layer(self):
        return (self.tid >> 8) & 0x3F

    @property
    def part(self):
        return self.tid >> 14


@dataclass
class Matrix:
    """One weight matrix as the kernels take it: the MMCF bytes unchanged."""
    kind: str            # 'q8' | 'q4' | 't3'
    rows: int
    cols: int
    body: np.ndarray     # uint8
    scale: float         # record scale (q8 ws, q4 ps, t3 unit)
    prebiased: bool = True
    plane: np.ndarray = None   # part 3 (f32 rows)
    s16: np.ndarray = None     # part 1 (q4)
    m16: np.ndarray = None     # part 2 (q4)
    scale_mul: float = 1.0     # 2^k of metadata key 15 (w2 only)

    def slice_rows(self, r0, r1):
        if self.kind == "q8":
            return Matrix("q8", r1 - r0, self.cols, self.body.reshape(self.rows, self.cols)[r0:r1].reshape(-1),
                          self.scale, self.prebiased,
                          None if self.plane is None else self.plane[r0:r1], scale_mul=self.scale_mul)
        if self.kind == "q4":
            g = self.cols // 32
            return Matrix("q4", r1 - r0, self.cols,
                          self.body.reshape(self.rows, self.cols // 2)[r0:r1].reshape(-1), self.scale,
                          s16=self.s16.reshape(self.rows, g)[r0:r1].reshape(-1),
                          m16=self.m16.reshape(self.rows, g)[r0:r1].reshape(-1), scale_mul=self.scale_mul)
        if r0 % 2:
            raise ValueError("t3 row slices start on a row pair")
        stride = (self.cols // 8) * 4
        rp = (r1 - r0 + 1) // 2
        return Matrix("t3", r1 - r0, self.cols,
                      self.body[(r0 // 2) * stride:(r0 // 2 + rp) * stride], self.scale,
                      plane=self.plane[r0:r1], scale_mul=self.scale_mul)

    def slice_cols(self, c0, c1):
        """A column range with the same scales (Model::slice_cols,
        engine/src/model.cpp:1700-1758): q4 on group boundaries, t3 on texels."""
        if self.kind == "q8":
            body = np.ascontiguousarray(self.body.reshape(self.rows, self.cols)[:, c0:c1]).reshape(-1)
            return Matrix("q8", self.rows, c1 - c0, body, self.scale, self.prebiased, self.plane,
                          scale_mul=self.scale_mul)
        if self.kind == "q4":
            if c0 % 32 or c1 % 32:
                raise ValueError("q4 column slices fall on 32-column groups")
            g = self.cols // 32
            body = np.ascontiguousarray(self.body.reshape(self.rows, self.cols // 2)[:, c0 // 2:c1 // 2]).reshape(-1)
            s16 = np.ascontiguousarray(self.s16.reshape(self.rows, g)[:, c0 // 32:c1 // 32]).reshape(-1)
            m16 = np.ascontiguousarray(self.m16.reshape(self.rows, g)[:, c0 // 32:c1 // 32]).reshape(-1)
            return Matrix("q4", self.rows, c1 - c0, body, self.scale, s16=s16, m16=m16, scale_mul=self.scale_mul)
        if c0 % 8 or c1 % 8:
            raise ValueError("t3 column slices fall on 8-column texels")
        body = self.body.reshape((self.rows + 1) // 2, self.cols // 8, 4)[:, c0 // 8:c1 // 8]
        return Matrix("t3", self.rows, c1 - c0, np.ascontiguousarray(body).reshape(-1), self.scale,
                      plane=self.plane, scale_mul=self.scale_mul)



class Container:
    """A parsed MMCF file: metadata and the tensor table, bodies borrowed."""

    def __init__(self, data):
        self.raw = memoryview(data)
        if bytes(self.raw[:4]) != MAGIC:
            raise ValueError("not an MMCF container")
        (ver, hsz, n, caps, moff, msize, doff, fsize) = struct.unpack_from("<HHIIIIQQ", self.raw, 4)
        if ver != 2 or hsz != HEADER_SIZE:
            raise ValueError("unsupported MMCF version %d" % ver)
        hcrc = struct.unpack_from("<I", self.raw, 40)[0]
        if hcrc and hcrc != (zlib.crc32(bytes(self.raw[:40])) & 0xFFFFFFFF):
            raise ValueError("header crc mismatch")
        if fsize != len(self.raw):
            raise ValueError("file size field %d != %d (truncated?)" % (fsize, len(self.raw)))
        self.meta = {}
        p = moff
        while p + 8 <= moff + msize:
            key, typ, ln = struct.unpack_from("<HHI", self.raw, p)
            self.meta[key] = bytes(self.raw[p + 8:p + 8 + ln])
            p += 8 + ln
        table = doff - n * REC_SIZE_V2
        self.records = []
        for i in range(n):
            o = table + i * REC_SIZE_V2
            tid, dt, _fl, group, _pad = struct.unpack_from("<HBBBB", self.raw, o)
            rows, cols = struct.unpack_from("<II", self.raw, o + 6)
            off, blen = struct.unpack_from("<QQ", self.raw, o + 14)
            crc, = struct.unpack_from("<I", self.raw, o + 30)
            scale, = struct.unpack_from("<f", self.raw, o + 34)
            body = self.raw[doff + off:doff + off + blen]
            if (zlib.crc32(body) & 0xFFFFFFFF) != crc:
                raise ValueError("tensor 0x%x: body crc mismatch" % tid)
            self.records.append(Record(tid, dt, group, rows, cols, scale, body))
        self.by_id = {r.tid: r for r in self.records}
        d = struct.unpack("<7i", self.meta[1])
        th, half, qk, _ = struct.unpack("<fBBH", self.meta[2])
        self.scheme = {v: k for k, v in SCHEMES.items()}[self.meta[3][0]]
        types = ["conv" if b else "attn" for b in self.meta.get(14, b"")]
        hid = list(self.meta.get(15, b""))
        eps = struct.unpack("<f", self.meta[11])[0] if 11 in self.meta else None
        self.spec = ModelSpec(*d, theta=th, rope_half=bool(half), qk_norm=bool(qk), layer_types=types,
                              hid_scale=hid, rms_eps=eps)

    def f32(self, tid):
        r = self.by_id[tid]
        return np.frombuffer(r.body, np.float32).reshape(r.rows, r.cols)

    def matrix(self, kind, layer=0):
        base = kind | (layer << 8)
        r = self.by_id[base]
        plane = self.by_id.get(base | (3 << 14))
        p = None if plane is None else np.frombuffer(plane.body, np.float32).copy()
        body = np.frombuffer(r.body, np.uint8)
        if r.dtype in (DT_Q8U8, DT_Q8I8):
            return Matrix("q8", r.rows, r.cols, body, r.scale, r.dtype == DT_Q8U8, p)
        if r.dtype == DT_T3:
            return Matrix("t3", r.rows, r.cols, body, r.scale, plane=p)
        if r.dtype == DT_Q4:
            s16 = np.frombuffer(self.by_id[base | (1 << 14)].body, np.int16)
            m16 = np.frombuffer(self.by_id[base | (2 << 14)].body, np.int16)
            return Matrix("q4", r.rows, r.cols, body, r.scale, s16=s16, m16=m16)
        raise ValueError("tensor 0x%x: dtype %d is not a kernel matrix" % (base, r.dtype))

    def layer_mats(self, l):
        """qkv, wo, w1, w3, w2 of a layer (a fused w13 is split at its middle
        row, engine/src/model.cpp's read of T_W13); w2 carries key 15's 2^k."""
        s = self.spec
        out = {}
        if (T_QKV | (l << 8)) in self.by_id:
            out["qkv"] = self.matrix(T_QKV, l)
            out["wo"] = self.matrix(T_WO, l)
        if (T_W13 | (l << 8)) in self.by_id:
            w13 = self.matrix(T_W13, l)
            out["w1"], out["w3"] = w13.slice_rows(0, s.hidden), w13.slice_rows(s.hidden, 2 * s.hidden)
        else:
            out["w1"] = self.matrix(T_W1, l)
            out["w3"] = self.matrix(T_W3, l)
        out["w2"] = self.matrix(T_W2, l)
        if s.hid_scale and l < len(s.hid_scale) and s.hid_scale[l]:
            out["w2"].scale_mul = float(1 << s.hid_scale[l])
        return out

    def logits_tiles(self):
        """The head as <=1536-row tiles; a --head-dedup container renders them
        from the signed embedding rows with plane = row scale / max row scale
        (engine/src/model.cpp:1566-1586)."""
        tiles, i = [], 0
        while (T_LOGITS | (i << 8)) in self.by_id:
            tiles.append(self.matrix(T_LOGITS, i))
            i += 1
        if tiles:
            return tiles
        emb, es = self.embedding()
        unit = float(es.max())
        for st in range(0, self.spec.vocab, LOGITS_GRID):
            rows = min(LOGITS_GRID, self.spec.vocab - st)
            body = np.ascontiguousarray(emb[st:st + rows]).view(np.uint8).reshape(-1)
            plane = (es[st:st + rows] / np.float32(unit)).astype(np.float32)
            tiles.append(Matrix("q8", rows, self.spec.dim, body, unit, False, plane))
        return tiles

    def embedding(self):
        r = self.by_id[T_EMB]
        return (np.frombuffer(r.body, np.int8).reshape(r.rows, r.cols),
                np.frombuffer(self.by_id[T_EMB_SCALE].body, np.float32))


def ffn_chunk(hidden):
    """Model::split_ffn (engine/src/model.cpp:246-266): a hidden over 2048 runs
    as two chunks of ceil(hidden/2); w2's column halves are two residual adds."""
    return (hidden + 1) // 2 if hidden > 2048 else 0
