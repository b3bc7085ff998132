"""ctypes binding of libvgx (include/vgx.h).

The library is the product: nothing here computes.  Loading fails loudly when
lib/libvgx.so has not been built -- there is no fallback path.
"""
import ctypes
import os

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# VGX_LIB names another build of the same library (e.g. one built with other
# compiler flags); by default the in-tree build.
LIB_PATH = os.environ.get("VGX_LIB") or os.path.join(PKG, "lib", "libvgx.so")

VGX_OK, VGX_EINVAL, VGX_EHIP, VGX_ENOMEM, VGX_ESTATE, VGX_ERANGE = 0, -1, -2, -3, -4, -5
Q8, Q4, T3 = 1, 2, 3
KIND = {"q8": Q8, "q4": Q4, "t3": T3}


class VgxError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__("vgx status %d: %s" % (status, msg))
        self.status = status


class WeightDesc(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("rows", ctypes.c_int), ("cols", ctypes.c_int),
                ("body", ctypes.c_void_p), ("body_bytes", ctypes.c_size_t), ("prebiased", ctypes.c_int),
                ("scale", ctypes.c_float), ("row_plane", ctypes.c_void_p), ("q4_scale", ctypes.c_void_p),
                ("q4_min", ctypes.c_void_p), ("scale_mul", ctypes.c_float)]


class AttnDesc(ctypes.Structure):
    _fields_ = [("dim", ctypes.c_int), ("heads", ctypes.c_int), ("kv_heads", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("seq", ctypes.c_int), ("layers", ctypes.c_int),
                ("kv_bits", ctypes.c_int), ("rope_half", ctypes.c_int), ("qk_norm", ctypes.c_int),
                ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p), ("q_norm", ctypes.c_void_p),
                ("k_norm", ctypes.c_void_p), ("layer_is_attn", ctypes.c_void_p)]


_P = ctypes.c_void_p
_I = ctypes.c_int
_SIGS = {
    "vgx_abi_version": (_I, []),
    "vgx_strerror": (ctypes.c_char_p, [_I]),
    "vgx_last_error": (ctypes.c_char_p, []),
    "vgx_ctx_create": (_I, [_I, ctypes.POINTER(_P)]),
    "vgx_ctx_destroy": (_I, [_P]),
    "vgx_ctx_set_stream": (_I, [_P, _P]),
    "vgx_ctx_stream": (_P, [_P]),
    "vgx_ctx_sync": (_I, [_P]),
    "vgx_mat_upload": (_I, [_P, ctypes.POINTER(WeightDesc), ctypes.POINTER(_P)]),
    "vgx_mat_clone": (_I, [_P, _P, ctypes.POINTER(_P)]),
    "vgx_mat_concat": (_I, [_P, _I, ctypes.POINTER(_P), ctypes.POINTER(_P)]),
    "vgx_argmax_rows": (_I, [_P, _I, _I, _P, _P]),
    "vgx_logits_chunks": (_I, [_P, _P, _I, ctypes.c_float, _P]),
    "vgx_mat_free": (_I, [_P]),
    "vgx_mat_shape": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "vgx_mat_weight_bytes": (ctypes.c_size_t, [_P]),
    "vgx_dequant": (_I, [_P, _P, _P]),
    "vgx_gemv": (_I, [_P, _P, _P, _P, _P]),
    "vgx_gemv_f32": (_I, [_P, _P, _P, _P]),
    "vgx_gemv_add_split": (_I, [_P, _P, _I, _P, _P, _P]),
    "vgx_group_create": (_I, [_P, _I, ctypes.POINTER(_P), ctypes.POINTER(_P)]),
    "vgx_group_free": (_I, [_P]),
    "vgx_group_rows": (_I, [_P]),
    "vgx_gemv_plan_info": (_I, [_P, _P, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "vgx_group_plan_info": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "vgx_gemv_group": (_I, [_P, _P, _P, _P]),
    "vgx_gemv_group_f32": (_I, [_P, _P, _P, _P]),
    "vgx_logits_argmax": (_I, [_P, _P, _P, _P, _P]),
    "vgx_ffn_gate": (_I, [_P, _P, _P, _P, _I, _P]),
    "vgx_rmsnorm": (_I, [_P, _I, _P, _P, ctypes.c_float, _P]),
    "vgx_gemv_rms": (_I, [_P, _P, _P, _P, ctypes.c_float, _P, _P]),
    "vgx_ffn_gate_rms": (_I, [_P, _P, _P, _P, _P, ctypes.c_float, _I, _P]),
    "vgx_gemv_group_rms": (_I, [_P, _P, _P, _P, ctypes.c_float, _P]),
    "vgx_logits_argmax_rms": (_I, [_P, _P, _P, _P, ctypes.c_float, _P, _P]),
    "vgx_logits_argmax_rms_noalloc": (_I, [_P, _P, _P, _P, ctypes.c_float, _P, _P]),
    "vgx_gemm": (_I, [_P, _P, _I, _P, _P, _P]),
    "vgx_gemm_add_split": (_I, [_P, _P, _I, _I, _P, _P, _P]),
    "vgx_ffn_gate_batch": (_I, [_P, _P, _P, _I, _P, _I, _P]),
    "vgx_rmsnorm_batch": (_I, [_P, _I, _I, _P, _P, ctypes.c_float, _P]),
    "vgx_gemm_rms": (_I, [_P, _P, _I, _P, _P, ctypes.c_float, _P, _P]),
    "vgx_ffn_gate_batch_rms": (_I, [_P, _P, _P, _I, _P, _P, ctypes.c_float, _I, _P]),
    "vgx_embed_q8_batch": (_I, [_P, _P, _P, _I, _I, _I, _P, _P]),
    "vgx_embed_q8_rms_batch": (_I, [_P, _P, _P, _I, _I, _I, _P, _P, _P, ctypes.c_float, _P]),
    "vgx_gemm_norm": (_I, [_P, _P, _I, _P, _P, _P, _P, ctypes.c_float, _P]),
    "vgx_gemm_add_split_norm": (_I, [_P, _P, _I, _I, _P, _P, _P, _P, ctypes.c_float, _P]),
    "vgx_kv_append_batch": (_I, [_P, _I, _I, _I, _P]),
    "vgx_conv_create": (_I, [_P, _I, _I, _I, _P, _P, ctypes.POINTER(_P)]),
    "vgx_conv_free": (_I, [_P]),
    "vgx_conv_reset": (_I, [_P]),
    "vgx_conv_step": (_I, [_P, _I, _I, _P, _P]),
    "vgx_conv_state_read": (_I, [_P, _I, _P]),
    "vgx_conv_state_write": (_I, [_P, _I, _P]),
    "vgx_attn_decode_batch": (_I, [_P, _I, _I, _I, _P, _P]),
    "vgx_embed_q8": (_I, [_P, _P, _P, _I, _I, _P, _P]),
    "vgx_attn_create": (_I, [_P, ctypes.POINTER(AttnDesc), ctypes.POINTER(_P)]),
    "vgx_attn_free": (_I, [_P]),
    "vgx_kv_append": (_I, [_P, _I, _I, _P]),
    "vgx_attn_decode": (_I, [_P, _I, _I, _P, _P]),
    "vgx_attn_block": (_I, [_P, _I, _I, _P, _P]),
    "vgx_attn_create_seqs": (_I, [_P, _P, _I, ctypes.POINTER(_P)]),
    "vgx_attn_seq_view": (_I, [_P, _I, ctypes.POINTER(_P)]),
    "vgx_attn_block_seqs": (_I, [_P, _I, _I, _I, _P, _P]),
    "vgx_attn_block_at": (_I, [_P, _I, _P, _P, _P]),
    "vgx_decode_advance": (_I, [_P, _P, _P, _P, _I]),
    "vgx_logits_argmax_step": (_I, [_P, _P, _P, _P, ctypes.c_float, _P, _P, _P, _P, _I, _P, _P, _I, _I, _P]),
    "vgx_kv_row_bytes": (_I, [_P]),
    "vgx_kv_read_rows": (_I, [_P, _I, _I, _I, _P]),
    "vgx_kv_write_rows": (_I, [_P, _I, _I, _I, _P]),
    "vgx_quantize_act": (None, [_P, _I, _P]),
    "vgx_x_pack_i16_2": (None, [_P, _I, _P]),
}

_lib = None


def _share_hip_runtime():
    """Load torch's HIP runtime ahead of libvgx when torch is installed.

    torch's HIP libraries request `libamdhip64.so` from their own directory;
    libvgx requests `libamdhip64.so.7`, the soname that both runtimes carry.
    In that order libvgx binds to the runtime torch brought in. In the other
    order torch finds no loaded library named `libamdhip64.so`, maps a second
    copy of the runtime, and that copy cannot open the GPU that the first one
    holds: torch then reports that no HIP GPUs are available."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def load():
    """The loaded library; raises when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("libvgx is not built (%s): run `make -C vc4-gles2-inference_amd` "
                               "or __graft_entry__.build()" % LIB_PATH)
        _share_hip_runtime()
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return sorted(_SIGS)


def check(status):
    if status != VGX_OK:
        msg = load().vgx_last_error()
        raise VgxError(status, msg.decode() if msg else "")
    return status
