"""ctypes binding to libfa_hip.so (the C ABI in include/fa_hip.h).

Loading fails loudly: there is no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# FA_LIB_PATH names another build of the same C ABI (the launch-audit build
# of tests/audit, which runs the host code against a stand-in runtime)
LIB_PATH = os.environ.get("FA_LIB_PATH") or os.path.join(HERE, "libfa_hip.so")

FA_OK, FA_E_INVALID, FA_E_STATE, FA_E_DEVICE, FA_E_OOM, FA_E_UNSUPPORTED = range(6)
ACT = {"none": 0, "gelu": 1, "tanh": 2, "relu": 3, "silu": 4, "gelu_erf": 5}
W_F16, W_INT8, W_INT4 = 0, 1, 2


class FaError(RuntimeError):
    """A failed fa_* call; .code is the fa_status value."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class EncoderCfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("D", "DFF", "H", "HD", "layers", "dwK", "Csub", "Fsub", "melBins")]


class EncoderOpts(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("sub_pad_t", "sub_pad_b", "sub_pad_l", "sub_pad_r", "conv_causal", "att_chunk", "att_left", "att_right")]


_lib = None

T = C.c_uint64  # fa_tensor / fa_arena / fa_staged
P = C.c_void_p  # fa_ctx* / fa_encoder*
I = C.c_int
I32P = C.POINTER(C.c_int32)
F32P = C.POINTER(C.c_float)

# (name, restype, argtypes) for every entry point in include/fa_hip.h
SIGNATURES = [
    ("fa_ctx_create", I, [I, C.POINTER(P)]),
    ("fa_ctx_destroy", None, [P]),
    ("fa_last_error", C.c_char_p, [P]),
    ("fa_version", C.c_char_p, []),
    ("fa_sync", I, [P]),
    ("fa_upload", I, [P, F32P, I, I, C.POINTER(T)]),
    ("fa_upload_f16", I, [P, F32P, I, I, C.POINTER(T)]),
    ("fa_alloc", I, [P, I, I, C.POINTER(T)]),
    ("fa_alloc_f16", I, [P, I, I, C.POINTER(T)]),
    ("fa_upload_f16_rows", I, [P, F32P, I, I, C.POINTER(T)]),
    ("fa_upload_bytes", I, [P, C.c_void_p, C.c_size_t, C.POINTER(T)]),
    ("fa_free_tensor", I, [P, T]),
    ("fa_pin", I, [P, T, I]),
    ("fa_push_arena", I, [P, C.POINTER(T)]),
    ("fa_pop_arena", I, [P, T]),
    ("fa_trim_pool", I, [P, C.c_size_t]),
    ("fa_tensor_info", I, [P, T, C.POINTER(I), C.POINTER(I), C.POINTER(I)]),
    ("fa_pool_info", I, [P, C.POINTER(C.c_size_t), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    ("fa_download", I, [P, T, F32P]),
    ("fa_stage_download", I, [P, T, C.POINTER(T)]),
    ("fa_staged_read", I, [P, T, F32P]),
    ("fa_rows_view", I, [P, T, I, C.POINTER(T)]),
    ("fa_begin_batch", I, [P]),
    ("fa_end_batch", I, [P]),
    ("fa_batch_open", I, [P]),
    ("fa_matmul", I, [P, T, T, T, I, T, C.POINTER(T)]),
    ("fa_matmul_pair", I, [P, T, T, T, T, T, C.POINTER(T)]),
    ("fa_matmul_int8", I, [P, T, T, T, I, I, T, I, C.POINTER(T)]),
    ("fa_matmul_nbits", I, [P, T, T, T, T, I, I, C.POINTER(T)]),
    ("fa_layernorm", I, [P, T, T, T, C.c_float, C.POINTER(T)]),
    ("fa_softmax", I, [P, T, C.POINTER(T)]),
    ("fa_conv1d", I, [P, T, T, I, I, T, I, I, I, I, I, I, C.POINTER(T)]),
    ("fa_conv2d", I, [P, T, T, I, I, I, I, I, I, T, I, I, I, I, I, I, I, I, C.POINTER(T)]),
    ("fa_bmm_qk", I, [P, T, T, T, I, I, I, I, C.POINTER(T)]),
    ("fa_bmm_pv", I, [P, T, T, I, I, I, C.POINTER(T)]),
    ("fa_rel_shift", I, [P, T, C.POINTER(T)]),
    ("fa_rel_shift_b", I, [P, T, I, C.POINTER(T)]),
    ("fa_rel_shift_stream", I, [P, T, I, I, I, I, I, I, I, I, I, C.POINTER(T)]),
    ("fa_attn_fused", I, [P, T, T, T, T, T, T, I, I, I, C.POINTER(T)]),
    ("fa_ewise", I, [P, T, T, I, C.POINTER(T)]),
    ("fa_scale", I, [P, T, C.c_float, C.POINTER(T)]),
    ("fa_silu", I, [P, T, C.POINTER(T)]),
    ("fa_relu", I, [P, T, C.POINTER(T)]),
    ("fa_glu", I, [P, T, C.POINTER(T)]),
    ("fa_transpose", I, [P, T, C.POINTER(T)]),
    ("fa_slice_cols", I, [P, T, I, I, C.POINTER(T)]),
    ("fa_set_cols", I, [P, T, T, I]),
    ("fa_slice_rows", I, [P, T, I, I, C.POINTER(T)]),
    ("fa_copy_rows", I, [P, T, T, I]),
    ("fa_concat_rows", I, [P, C.POINTER(T), I, C.POINTER(T)]),
    ("fa_sub_reshape", I, [P, T, I, I, I, C.POINTER(T)]),
    ("fa_row_bias_act", I, [P, T, T, I, C.POINTER(T)]),
    ("fa_profile_start", I, [P, I]),
    ("fa_profile_end", I, [P, I, C.c_void_p, F32P, C.POINTER(I)]),
    ("fa_profile_only", I, [P, C.c_char_p]),
    ("fa_dequant_int8", I, [P, T, T, I, I, C.POINTER(T)]),
    ("fa_dequant_int4", I, [P, T, T, I, I, C.POINTER(T)]),
    ("fa_quantize_weights", I, [I, F32P, I, I, C.c_void_p, C.c_void_p]),
    ("fa_gemv_quant", I, [P, T, T, T, I, I, I, C.POINTER(T)]),
    ("fa_gemv_quant_batch", I, [P, I, C.POINTER(T), C.POINTER(T), C.POINTER(T), I, I, I, C.POINTER(T)]),
    ("fa_pack_windows", I, [P, T, I32P, I32P, I, I, C.POINTER(T)]),
    ("fa_mel_windows", I, [P, T, I32P, I32P, I, I, C.c_double, I, C.POINTER(T)]),
    ("fa_leaky_relu", I, [P, T, C.c_double, C.POINTER(T)]),
    ("fa_snake", I, [P, T, T, C.POINTER(T)]),
    ("fa_adain", I, [P, T, T, T, C.c_double, C.POINTER(T)]),
    ("fa_im2col", I, [P, T, I, I, I, I, C.POINTER(T)]),
    ("fa_conv_transpose1d", I, [P, T, T, I, I, T, I, I, I, I, I, I, C.POINTER(T)]),
    ("fa_gather_cols", I, [P, T, C.POINTER(C.c_uint32), I, C.POINTER(T)]),
    ("fa_lstm", I, [P, T, T, T, T, I, C.POINTER(T)]),
    ("fa_jbatch", I, [P, T, I, I, T, I, C.POINTER(T)]),
    ("fa_argmax_rows", I, [P, T, I, I, I, C.POINTER(T)]),
    ("fa_joint_argmax", I, [P, T, I, I, T, T, T, I, I, I, C.POINTER(T)]),
    ("fa_mel_windows_static", I, [P, C.c_void_p, C.c_int64, I32P, I32P, I, I, C.c_double, I, C.c_void_p, C.c_int64]),
    ("fa_tdt_load", I, [P, C.POINTER(C.POINTER(C.c_float)), C.POINTER(P)]),
    ("fa_tdt_destroy", None, [P]),
    ("fa_tdt_decode", I, [P, T, I32P, I, I, I32P, I32P, I32P]),
    ("fa_transcribe_groups", I, [P, P, P, T, I, I32P, I32P, I32P, T, T, I, C.c_double, I, I, I32P, I32P, I32P, I32P]),
    ("fa_window_row_map", I, [P, I32P, I, I, I, I32P, C.POINTER(I)]),
    ("fa_encoder_load", I, [P, C.POINTER(EncoderCfg), I, C.POINTER(C.c_char_p), C.POINTER(F32P), C.POINTER(C.c_int64), I, I, C.POINTER(P)]),
    ("fa_encoder_destroy", None, [P]),
    ("fa_encoder_set_exact", I, [P, I, I, C.c_uint]),
    ("fa_encoder_get_exact", I, [P, I]),
    ("fa_encoder_load_opts", I, [P, C.POINTER(EncoderCfg), C.POINTER(EncoderOpts), I, C.POINTER(C.c_char_p), C.POINTER(F32P), C.POINTER(C.c_int64), I, I,
                                 C.POINTER(P)]),
    ("fa_encoder_forward", I, [P, P, T, I32P, I, I, I, C.POINTER(T)]),
    ("fa_encoder_forward_stream", I, [P, P, T, I32P, I32P, I, I, I, C.POINTER(T)]),
    ("fa_encoder_forward_stream_batches", I, [P, P, T, I, I32P, I32P, I32P, I, I, C.POINTER(T)]),
    ("fa_encoder_tsub", I, [I]),
    ("fa_encoder_tsub_of", I, [P, I]),
    ("fa_stream_create", I, [P, P, I, I, C.POINTER(P)]),
    ("fa_stream_push", I, [P, F32P, I, C.POINTER(T)]),
    ("fa_stream_push_many", I, [I, C.POINTER(P), C.POINTER(F32P), C.POINTER(I), C.POINTER(T)]),
    ("fa_stream_flush", I, [P, C.POINTER(T)]),
    ("fa_stream_destroy", None, [P]),
]


def lib() -> C.CDLL:
    """The loaded library (raises if libfa_hip.so was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python fluidaudio-web_amd/csrc/build.py` "
                               "(or __graft_entry__.build()); there is no CPU fallback")
        L = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(ctx_ptr, status: int) -> None:
    if status != FA_OK:
        msg = lib().fa_last_error(ctx_ptr) if ctx_ptr else b""
        raise FaError(status, (msg or b"").decode() or f"fa status {status}")
