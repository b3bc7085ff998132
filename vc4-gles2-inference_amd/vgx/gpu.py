"""Host-side mirror of the reference engine's GPU object over libvgx.

`GPU` has the reference's entry points (engine/src/gpu.h:41-633: upload,
matvec / matvec_add, ffn_split_chunked, rmsnorm, attention_block,
kv_rope_write, logits_from) with the same argument meaning; device buffers are
torch tensors on the GPU (plumbing only: every number is computed by libvgx).
"""
import ctypes

import numpy as np
import torch

from . import lib as _l
from .mmcf import Matrix


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _np_ptr(a):
    return ctypes.c_void_p(0 if a is None else a.ctypes.data)


class Mat:
    """An uploaded weight matrix (GPU::upload's result)."""

    def __init__(self, gpu, handle, m):
        self.gpu, self.h, self.rows, self.cols, self.kind = gpu, handle, m.rows, m.cols, m.kind

    @property
    def weight_bytes(self):
        return int(_l.load().vgx_mat_weight_bytes(self.h))

    def free(self):
        if self.h:
            _l.load().vgx_mat_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Group:
    """Matrices sharing one input, launched as one kernel (logits tiles)."""

    def __init__(self, gpu, mats):
        L = _l.load()
        arr = (ctypes.c_void_p * len(mats))(*[m.h for m in mats])
        h = ctypes.c_void_p()
        _l.check(L.vgx_group_create(gpu.ctx, len(mats), arr, ctypes.byref(h)))
        self.gpu, self.h, self.mats = gpu, h, list(mats)
        self.rows = int(L.vgx_group_rows(h))

    def gemv(self, x, out=None):
        out = out if out is not None else torch.empty(self.rows, dtype=torch.int16, device=x.device)
        _l.check(_l.load().vgx_gemv_group(self.gpu.ctx, self.h, _ptr(x), _ptr(out)))
        return out

    def plan(self):
        """(lanes per row, rows per lane) of this group's launch."""
        lpr, ri = ctypes.c_int(), ctypes.c_int()
        _l.check(_l.load().vgx_group_plan_info(self.h, ctypes.byref(lpr), ctypes.byref(ri)))
        return lpr.value, ri.value

    def gemv_f32(self, x, out=None):
        out = out if out is not None else torch.empty(self.rows, dtype=torch.float32, device=x.device)
        _l.check(_l.load().vgx_gemv_group_f32(self.gpu.ctx, self.h, _ptr(x), _ptr(out)))
        return out

    def logits_argmax(self, x, logits=None, token=None):
        logits = logits if logits is not None else torch.empty(self.rows, dtype=torch.int16, device=x.device)
        token = token if token is not None else torch.empty(1, dtype=torch.int32, device=x.device)
        _l.check(_l.load().vgx_logits_argmax(self.gpu.ctx, self.h, _ptr(x), _ptr(logits), _ptr(token)))
        return logits, token

    def gemv_rms(self, x, rms_w, eps, out=None):
        """rmsnorm(x, rms_w, eps) then the group GEMV, one launch."""
        out = out if out is not None else torch.empty(self.rows, dtype=torch.int16, device=x.device)
        _l.check(_l.load().vgx_gemv_group_rms(self.gpu.ctx, self.h, _ptr(x), _ptr(rms_w), float(eps), _ptr(out)))
        return out

    def logits_argmax_rms(self, x, rms_w, eps, logits=None, token=None):
        """The final norm, the logits pass and the argmax in one launch."""
        logits = logits if logits is not None else torch.empty(self.rows, dtype=torch.int16, device=x.device)
        token = token if token is not None else torch.empty(1, dtype=torch.int32, device=x.device)
        _l.check(_l.load().vgx_logits_argmax_rms(self.gpu.ctx, self.h, _ptr(x), _ptr(rms_w), float(eps),
                                                  _ptr(logits), _ptr(token)))
        return logits, token

    def logits_argmax_step(self, x, rms_w, eps, logits, token, pos, hist, emb, emb_scale, x_next):
        """logits_argmax_rms, then in the reduction launch hist[pos + 1] =
        token, ++pos and the token's q8 embedding row into x_next."""
        vocab, dim = emb.shape
        _l.check(_l.load().vgx_logits_argmax_step(self.gpu.ctx, self.h, _ptr(x), _ptr(rms_w), float(eps),
                                                   _ptr(logits), _ptr(token), _ptr(pos), _ptr(hist),
                                                   int(hist.numel()), _ptr(emb), _ptr(emb_scale), vocab, dim,
                                                   _ptr(x_next)))
        return logits, token

    def free(self):
        if self.h:
            _l.load().vgx_group_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Conv:
    """LFM2 conv-block state and taps (GPU::init_conv / set_conv_kernel)."""

    def __init__(self, gpu, w, layer_is_conv=None):
        L = _l.load()
        self._w = np.ascontiguousarray(w, np.float32)  # [layers][dim][3]
        layers, dim, k = self._w.shape
        self._types = None if layer_is_conv is None else np.ascontiguousarray(layer_is_conv, np.uint8)
        h = ctypes.c_void_p()
        _l.check(L.vgx_conv_create(gpu.ctx, dim, layers, k, _np_ptr(self._w), _np_ptr(self._types),
                                   ctypes.byref(h)))
        self.gpu, self.h, self.dim = gpu, h, dim

    def step(self, layer, bcx, out=None):
        """bcx: (ntok, 3*dim) or (3*dim,) q16; returns y of the same leading shape."""
        n = 1 if bcx.dim() == 1 else bcx.shape[0]
        shape = (self.dim,) if bcx.dim() == 1 else (n, self.dim)
        out = out if out is not None else torch.empty(shape, dtype=torch.int16, device=bcx.device)
        _l.check(_l.load().vgx_conv_step(self.h, layer, n, _ptr(bcx), _ptr(out)))
        return out

    def reset(self):
        _l.check(_l.load().vgx_conv_reset(self.h))

    def state(self, layer):
        buf = np.empty((2, self.dim), np.int16)
        _l.check(_l.load().vgx_conv_state_read(self.h, layer, _np_ptr(buf)))
        return buf

    def set_state(self, layer, st):
        st = np.ascontiguousarray(st, np.int16)
        _l.check(_l.load().vgx_conv_state_write(self.h, layer, _np_ptr(st)))

    def free(self):
        if self.h:
            _l.load().vgx_conv_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Attention:
    """GPU::init_attention's state: KV cache, RoPE table, q/k norm weights."""

    def __init__(self, gpu, dim, heads, kv_heads, head_dim, seq, layers, kv_bits, rope_half, qk_norm,
                 rope_cos, rope_sin, q_norm=None, k_norm=None, layer_is_attn=None, nseq=1):
        L = _l.load()
        self._keep = [np.ascontiguousarray(rope_cos, np.float32), np.ascontiguousarray(rope_sin, np.float32),
                      None if q_norm is None else np.ascontiguousarray(q_norm, np.float32),
                      None if k_norm is None else np.ascontiguousarray(k_norm, np.float32),
                      None if layer_is_attn is None else np.ascontiguousarray(layer_is_attn, np.uint8)]
        d = _l.AttnDesc(dim, heads, kv_heads, head_dim, seq, layers, kv_bits, int(rope_half), int(qk_norm),
                        _np_ptr(self._keep[0]), _np_ptr(self._keep[1]), _np_ptr(self._keep[2]),
                        _np_ptr(self._keep[3]), _np_ptr(self._keep[4]))
        h = ctypes.c_void_p()
        _l.check(L.vgx_attn_create_seqs(gpu.ctx, ctypes.byref(d), nseq, ctypes.byref(h)))
        self.gpu, self.h, self.dim, self.seq, self.nseq = gpu, h, dim, seq, nseq
        self.row_bytes = int(L.vgx_kv_row_bytes(h))
        self.views = []

    def view(self, s):
        """Sequence s's cache as a single-sequence Attention (freed with the parent)."""
        h = ctypes.c_void_p()
        _l.check(_l.load().vgx_attn_seq_view(self.h, s, ctypes.byref(h)))
        v = Attention.__new__(Attention)
        v.gpu, v.h, v.dim, v.seq, v.nseq, v.row_bytes, v.views = self.gpu, h, self.dim, self.seq, 1, self.row_bytes, []
        self.views.append(v)
        return v

    def block_seqs(self, layer, pos, qkv, out=None):
        """Position pos of the sequences 0..n-1 for the n rows of qkv."""
        n = qkv.shape[0]
        out = out if out is not None else torch.empty((n, self.dim), dtype=torch.int16, device=qkv.device)
        _l.check(_l.load().vgx_attn_block_seqs(self.h, layer, pos, n, _ptr(qkv), _ptr(out)))
        return out

    def kv_append(self, layer, pos, qkv):
        _l.check(_l.load().vgx_kv_append(self.h, layer, pos, _ptr(qkv)))

    def decode(self, layer, pos, qkv, out=None):
        out = out if out is not None else torch.empty(self.dim, dtype=torch.int16, device=qkv.device)
        _l.check(_l.load().vgx_attn_decode(self.h, layer, pos, _ptr(qkv), _ptr(out)))
        return out

    def block(self, layer, pos, qkv, out=None):
        out = out if out is not None else torch.empty(self.dim, dtype=torch.int16, device=qkv.device)
        _l.check(_l.load().vgx_attn_block(self.h, layer, pos, _ptr(qkv), _ptr(out)))
        return out

    def block_batch(self, layer, pos0, qkv, out=None):
        """Positions pos0 .. pos0 + n - 1 for the n rows of qkv: the KV rows
        are appended first, then every position attends to its prefix."""
        n = qkv.shape[0]
        out = out if out is not None else torch.empty((n, self.dim), dtype=torch.int16, device=qkv.device)
        L = _l.load()
        _l.check(L.vgx_kv_append_batch(self.h, layer, pos0, n, _ptr(qkv)))
        _l.check(L.vgx_attn_decode_batch(self.h, layer, pos0, n, _ptr(qkv), _ptr(out)))
        return out

    def read_rows(self, layer, row0, nrows):
        buf = np.empty(nrows * self.row_bytes, np.uint8)
        _l.check(_l.load().vgx_kv_read_rows(self.h, layer, row0, nrows, _np_ptr(buf)))
        return buf

    def write_rows(self, layer, row0, data):
        data = np.ascontiguousarray(data, np.uint8)
        _l.check(_l.load().vgx_kv_write_rows(self.h, layer, row0, data.size // self.row_bytes, _np_ptr(data)))

    def free(self):
        for v in getattr(self, "views", []):
            v.free()
        if self.h:
            _l.load().vgx_attn_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class GPU:
    """One libvgx context on one device, issuing on torch's current stream."""

    def __init__(self, device=0):
        L = _l.load()
        h = ctypes.c_void_p()
        _l.check(L.vgx_ctx_create(device, ctypes.byref(h)))
        self.ctx, self.device = h, torch.device("cuda", device)
        self.use_torch_stream()

    def use_torch_stream(self):
        s = torch.cuda.current_stream(self.device).cuda_stream
        _l.check(_l.load().vgx_ctx_set_stream(self.ctx, ctypes.c_void_p(s)))

    def sync(self):
        _l.check(_l.load().vgx_ctx_sync(self.ctx))

    # -- weights
    def upload(self, m: Matrix):
        keep = [np.ascontiguousarray(m.body, np.uint8)]
        plane = s16 = m16 = None
        if m.plane is not None:
            plane = np.ascontiguousarray(m.plane, np.float32)
        if m.kind == "q4":
            s16 = np.ascontiguousarray(m.s16, np.int16)
            m16 = np.ascontiguousarray(m.m16, np.int16)
        d = _l.WeightDesc(_l.KIND[m.kind], m.rows, m.cols, _np_ptr(keep[0]), keep[0].size, int(m.prebiased),
                          float(m.scale), _np_ptr(plane), _np_ptr(s16), _np_ptr(m16), float(m.scale_mul))
        h = ctypes.c_void_p()
        _l.check(_l.load().vgx_mat_upload(self.ctx, ctypes.byref(d), ctypes.byref(h)))
        return Mat(self, h, m)

    def clone(self, mat):
        h = ctypes.c_void_p()
        _l.check(_l.load().vgx_mat_clone(self.ctx, mat.h, ctypes.byref(h)))
        c = Mat.__new__(Mat)
        c.gpu, c.h, c.rows, c.cols, c.kind = self, h, mat.rows, mat.cols, mat.kind
        return c

    def dequant(self, mat):
        out = torch.empty((mat.rows, mat.cols), dtype=torch.float32, device=self.device)
        _l.check(_l.load().vgx_dequant(self.ctx, mat.h, _ptr(out)))
        return out

    def group(self, mats):
        return Group(self, mats)

    def concat(self, mats):
        """One matrix with the rows of mats in order (q8 or t3, equal cols)."""
        arr = (ctypes.c_void_p * len(mats))(*[m.h for m in mats])
        h = ctypes.c_void_p()
        _l.check(_l.load().vgx_mat_concat(self.ctx, len(mats), arr, ctypes.byref(h)))
        c = Mat.__new__(Mat)
        c.gpu, c.h, c.rows, c.cols, c.kind = self, h, sum(m.rows for m in mats), mats[0].cols, mats[0].kind
        return c

    def argmax_rows(self, v, out=None):
        """The first maximum of each row of a 2-D int16 tensor."""
        out = out if out is not None else torch.empty(v.shape[0], dtype=torch.int32, device=v.device)
        _l.check(_l.load().vgx_argmax_rows(self.ctx, v.shape[0], v.shape[1], _ptr(v), _ptr(out)))
        return out

    def logits_chunks(self, logits, temp):
        """The candidate pass over a q16 logits row: an int32 tensor of
        ceil(n / 16) x 6 chunk records (v1, i1, v2, i2, max, sum on 1/2048)."""
        n = logits.numel()
        out = torch.empty(((n + 15) // 16, 6), dtype=torch.int32, device=logits.device)
        _l.check(_l.load().vgx_logits_chunks(self.ctx, _ptr(logits), n, float(temp), _ptr(out)))
        return out

    # -- GEMV family
    def matvec(self, mat, x, res=None, out=None):
        """matvec_to / matvec_add: y = q16(W.x [+ res])."""
        out = out if out is not None else torch.empty(mat.rows, dtype=torch.int16, device=x.device)
        _l.check(_l.load().vgx_gemv(self.ctx, mat.h, _ptr(x), _ptr(res), _ptr(out)))
        return out

    def plan(self, mat):
        """(lanes per row, rows per lane) of a GEMV launch over mat."""
        lpr, ri = ctypes.c_int(), ctypes.c_int()
        _l.check(_l.load().vgx_gemv_plan_info(self.ctx, mat.h, ctypes.byref(lpr), ctypes.byref(ri)))
        return lpr.value, ri.value

    def matvec_f32(self, mat, x, out=None):
        out = out if out is not None else torch.empty(mat.rows, dtype=torch.float32, device=x.device)
        _l.check(_l.load().vgx_gemv_f32(self.ctx, mat.h, _ptr(x), _ptr(out)))
        return out

    def matvec_add_split(self, mat, split, x, res, out=None):
        """matvec_add(w2a) then matvec_add(w2b) over the column halves."""
        out = out if out is not None else torch.empty(mat.rows, dtype=torch.int16, device=x.device)
        _l.check(_l.load().vgx_gemv_add_split(self.ctx, mat.h, split, _ptr(x), _ptr(res), _ptr(out)))
        return out

    def ffn_gate(self, w1, w3, x, hs=0, out=None):
        out = out if out is not None else torch.empty(w1.rows, dtype=torch.int16, device=x.device)
        _l.check(_l.load().vgx_ffn_gate(self.ctx, w1.h, w3.h, _ptr(x), hs, _ptr(out)))
        return out

    def rmsnorm(self, x, w, eps=1e-5, out=None):
        out = out if out is not None else torch.empty_like(x)
        _l.check(_l.load().vgx_rmsnorm(self.ctx, x.numel(), _ptr(x), _ptr(w), float(eps), _ptr(out)))
        return out

    # -- batched prefill: x is (ntok, cols), outputs (ntok, rows)
    def gemm(self, mat, x, res=None, out=None):
        n = x.shape[0]
        out = out if out is not None else torch.empty((n, mat.rows), dtype=torch.int16, device=x.device)
        _l.check(_l.load().vgx_gemm(self.ctx, mat.h, n, _ptr(x), _ptr(res), _ptr(out)))
        return out

    def gemm_add_split(self, mat, split, x, res, out=None):
        n = x.shape[0]
        out = out if out is not None else torch.empty((n, mat.rows), dtype=torch.int16, device=x.device)
        _l.check(_l.load().vgx_gemm_add_split(self.ctx, mat.h, split, n, _ptr(x), _ptr(res), _ptr(out)))
        return out

    def ffn_gate_batch(self, w1, w3, x, hs=0, out=None):
        n = x.shape[0]
        out = out if out is not None else torch.empty((n, w1.rows), dtype=torch.int16, device=x.device)
        _l.check(_l.load().vgx_ffn_gate_batch(self.ctx, w1.h, w3.h, n, _ptr(x), hs, _ptr(out)))
        return out

    def gemm_norm(self, mat, x, res, rms_w, eps=1e-5, split=0):
        """gemm (or gemm_add_split when split) and the RMSNorm of the rows it
        wrote: (y, yn)."""
        n = x.shape[0]
        y = torch.empty((n, mat.rows), dtype=torch.int16, device=x.device)
        yn = torch.empty_like(y)
        L = _l.load()
        if split:
            _l.check(L.vgx_gemm_add_split_norm(self.ctx, mat.h, split, n, _ptr(x), _ptr(res), _ptr(y), _ptr(rms_w),
                                               float(eps), _ptr(yn)))
        else:
            _l.check(L.vgx_gemm_norm(self.ctx, mat.h, n, _ptr(x), _ptr(res), _ptr(y), _ptr(rms_w), float(eps),
                                     _ptr(yn)))
        return y, yn

    def gemm_rms(self, mat, x, rms_w, eps=1e-5, res=None, out=None):
        """rmsnorm_batch(x, rms_w, eps) then gemm, one launch."""
        n = x.shape[0]
        out = out if out is not None else torch.empty((n, mat.rows), dtype=torch.int16, device=x.device)
        _l.check(_l.load().vgx_gemm_rms(self.ctx, mat.h, n, _ptr(x), _ptr(rms_w), float(eps), _ptr(res), _ptr(out)))
        return out

    def ffn_gate_batch_rms(self, w1, w3, x, rms_w, eps=1e-5, hs=0, out=None):
        """rmsnorm_batch(x, rms_w, eps) then ffn_gate_batch, one launch."""
        n = x.shape[0]
        out = out if out is not None else torch.empty((n, w1.rows), dtype=torch.int16, device=x.device)
        _l.check(_l.load().vgx_ffn_gate_batch_rms(self.ctx, w1.h, w3.h, n, _ptr(x), _ptr(rms_w), float(eps), hs,
                                                  _ptr(out)))
        return out

    def rmsnorm_batch(self, x, w, eps=1e-5, out=None):
        out = out if out is not None else torch.empty_like(x)
        _l.check(_l.load().vgx_rmsnorm_batch(self.ctx, x.shape[0], x.shape[1], _ptr(x), _ptr(w), float(eps),
                                             _ptr(out)))
        return out

    def embed_q8_batch(self, emb, emb_scale, tokens, out=None):
        vocab, dim = emb.shape
        n = tokens.numel()
        out = out if out is not None else torch.empty((n, dim), dtype=torch.int16, device=emb.device)
        _l.check(_l.load().vgx_embed_q8_batch(self.ctx, _ptr(emb), _ptr(emb_scale), vocab, dim, n, _ptr(tokens),
                                              _ptr(out)))
        return out

    def embed_q8_rms_batch(self, emb, emb_scale, tokens, rms_w, eps=1e-5):
        """(embedding rows, their RMSNorm) of a batch of tokens, one launch."""
        vocab, dim = emb.shape
        n = tokens.numel()
        x = torch.empty((n, dim), dtype=torch.int16, device=emb.device)
        y = torch.empty((n, dim), dtype=torch.int16, device=emb.device)
        _l.check(_l.load().vgx_embed_q8_rms_batch(self.ctx, _ptr(emb), _ptr(emb_scale), vocab, dim, n, _ptr(tokens),
                                                  _ptr(x), _ptr(rms_w), ctypes.c_float(eps), _ptr(y)))
        return x, y

    def matvec_rms(self, mat, x, rms_w, eps=1e-5, res=None, out=None):
        """rmsnorm(x, rms_w, eps) then matvec_add, one launch."""
        out = out if out is not None else torch.empty(mat.rows, dtype=torch.int16, device=x.device)
        _l.check(_l.load().vgx_gemv_rms(self.ctx, mat.h, _ptr(x), _ptr(rms_w), float(eps), _ptr(res), _ptr(out)))
        return out

    def ffn_gate_rms(self, w1, w3, x, rms_w, eps=1e-5, hs=0, out=None):
        """rmsnorm(x, rms_w, eps) then the fused FFN gate, one launch."""
        out = out if out is not None else torch.empty(w1.rows, dtype=torch.int16, device=x.device)
        _l.check(_l.load().vgx_ffn_gate_rms(self.ctx, w1.h, w3.h, _ptr(x), _ptr(rms_w), float(eps), hs, _ptr(out)))
        return out

    def decode_advance(self, pos, token, hist):
        """hist[pos + 1] = token (inside hist), then ++pos; device scalars."""
        _l.check(_l.load().vgx_decode_advance(self.ctx, _ptr(pos), _ptr(token), _ptr(hist), int(hist.numel())))

    def embed_q8(self, emb, emb_scale, token, out=None):
        vocab, dim = emb.shape
        out = out if out is not None else torch.empty(dim, dtype=torch.int16, device=emb.device)
        _l.check(_l.load().vgx_embed_q8(self.ctx, _ptr(emb), _ptr(emb_scale), vocab, dim, _ptr(token), _ptr(out)))
        return out

    def attention(self, **kw):
        return Attention(self, **kw)

    def conv(self, w, layer_is_conv=None):
        return Conv(self, w, layer_is_conv)

    def close(self):
        if self.ctx:
            _l.load().vgx_ctx_destroy(self.ctx)
            self.ctx = None


def quantize_act(v):
    """quantize_act on the host (libvgx's helper)."""
    v = np.ascontiguousarray(v, np.float32).ravel()
    q = np.empty(v.size, np.int16)
    _l.load().vgx_quantize_act(_np_ptr(v), v.size, _np_ptr(q))
    return q


def x_pack_i16_2(v):
    v = np.ascontiguousarray(v, np.float32).ravel()
    out = np.empty(4 * ((v.size + 1) // 2), np.uint8)
    _l.load().vgx_x_pack_i16_2(_np_ptr(v), v.size, _np_ptr(out))
    return out
