"""ctypes binding of libmtl.so (the C ABI declared in include/mtl.h).

torch is imported before the library is opened: torch ships the HIP runtime
(SONAME libamdhip64.so.7) and libmtl.so must bind to that same loaded copy,
so streams and device pointers handed over by torch are valid inside it.

There is no fallback: if the library is missing or cannot be loaded, every
op raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded first, see module docstring)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmtl.so")
ABI_VERSION = 3

MTL_F32 = 0
MTL_BF16 = 1

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_vp = ctypes.c_void_p
_fp = ctypes.c_void_p  # device float*


class ScanParams(ctypes.Structure):
    """mirror of mtl_scan_params"""
    _fields_ = [
        ("u", _vp), ("u_sb", _i64), ("u_sd", _i64), ("u_sl", _i64),
        ("delta", _vp), ("delta_sb", _i64), ("delta_sd", _i64), ("delta_sl", _i64),
        ("z", _vp), ("z_sb", _i64), ("z_sd", _i64), ("z_sl", _i64),
        ("B", _vp), ("B_sb", _i64), ("B_sn", _i64), ("B_sl", _i64),
        ("C", _vp), ("C_sb", _i64), ("C_sn", _i64), ("C_sl", _i64),
        ("y", _vp), ("y_sb", _i64), ("y_sd", _i64), ("y_sl", _i64),
        ("A", _fp), ("D", _fp), ("delta_bias", _fp), ("h0", _fp), ("h_out", _fp),
        ("batch", _i64), ("seqlen", _i64), ("dim", _i64), ("dstate", _i64),
        ("dtype", _i32), ("delta_softplus", _i32), ("a_is_log", _i32), ("algo", _i32),
    ]


class ConvParams(ctypes.Structure):
    """mirror of mtl_conv_params"""
    _fields_ = [
        ("x", _vp), ("x_sb", _i64), ("x_sd", _i64), ("x_sl", _i64),
        ("out", _vp), ("out_sb", _i64), ("out_sd", _i64), ("out_sl", _i64),
        ("w", _fp), ("bias", _fp), ("conv_state_in", _vp), ("conv_state_out", _vp),
        ("batch", _i64), ("seqlen", _i64), ("dim", _i64),
        ("width", _i32), ("dtype", _i32), ("silu", _i32), ("reserved", _i32),
    ]


class PrefillLayer(ctypes.Structure):
    """mirror of mtl_prefill_layer"""
    _fields_ = [
        ("norm_w", _vp), ("eps", ctypes.c_float), ("reserved", _i32),
        ("W_in", _vp), ("b_in", _vp), ("conv_w", _vp), ("conv_b", _vp), ("W_x", _vp), ("W_dt", _vp),
        ("dt_bias", _vp), ("A_log", _vp), ("Dv", _vp), ("W_out", _vp), ("b_out", _vp),
        ("conv_state_in", _vp), ("conv_state_out", _vp), ("h0", _vp), ("h_out", _vp),
    ]


class PrefillShortArgs(ctypes.Structure):
    """mirror of mtl_prefill_short_args"""
    _fields_ = [
        ("h", _vp), ("xn", _vp), ("u", _vp), ("z", _vp), ("dt", _vp), ("y", _vp), ("x_parts", _vp),
        ("x_dbl", _vp), ("y_parts", _vp), ("norm_f", _vp), ("normed_out", _vp),
        ("eps_f", ctypes.c_float), ("d_conv", _i32), ("n_layers", _i32), ("reserved", _i32),
        ("batch", _i64), ("seqlen", _i64), ("d_model", _i64), ("d_inner", _i64), ("d_state", _i64),
        ("dt_rank", _i64),
    ]


class PrefillLongArgs(ctypes.Structure):
    """mirror of mtl_prefill_long_args"""
    _fields_ = [
        ("h", _vp), ("xn", _vp), ("xz", _vp), ("u", _vp), ("x_dbl", _vp), ("dt", _vp), ("y", _vp), ("out", _vp),
        ("blas_ws", _vp), ("blas_ws_bytes", _i64), ("norm_f", _vp), ("normed_out", _vp),
        ("eps_f", ctypes.c_float), ("d_conv", _i32), ("n_layers", _i32), ("skinny_rows", _i32),
        ("batch", _i64), ("seqlen", _i64), ("d_model", _i64), ("d_inner", _i64), ("d_state", _i64),
        ("dt_rank", _i64),
    ]


class DecodeLayer(ctypes.Structure):
    """mirror of mtl_decode_layer"""
    _fields_ = [
        ("norm_w", _vp), ("eps", ctypes.c_float), ("reserved", _i32),
        ("W_in", _vp), ("b_in", _vp), ("conv_w", _vp), ("conv_b", _vp), ("W_xT", _vp), ("W_x", _vp),
        ("W_dt", _vp), ("dt_bias", _vp), ("A_log", _vp), ("Dv", _vp), ("W_out", _vp), ("b_out", _vp),
        ("conv_state", _vp), ("ssm_state", _vp),
    ]


class DecodeStepArgs(ctypes.Structure):
    """mirror of mtl_decode_step_args"""
    _fields_ = [
        ("ids", _vp), ("emb", _vp), ("norm_f", _vp), ("logits", _vp), ("xc", _vp), ("gz", _vp), ("y", _vp),
        ("x0", _vp), ("x1", _vp), ("resid", _vp), ("xpart", _vp),
        ("eps_f", ctypes.c_float), ("vocab", _i32), ("n_layers", _i32), ("batch", _i32),
        ("d_model", _i32), ("d_inner", _i32), ("d_state", _i32), ("dt_rank", _i32), ("d_conv", _i32),
        ("channels_per_block", _i32), ("split_k", _i32), ("xproj_parts", _i32),
    ]


class DecodeStepBatchedArgs(ctypes.Structure):
    """mirror of mtl_decode_step_batched_args"""
    _fields_ = [
        ("h", _vp), ("normed_out", _vp), ("norm_f", _vp), ("inp", _vp), ("xn", _vp), ("xc", _vp), ("z", _vp),
        ("y", _vp), ("xpart", _vp), ("x_dbl", _vp), ("parts", _vp), ("sq", _vp), ("counters", _vp),
        ("eps_f", ctypes.c_float), ("n_layers", _i32), ("batch", _i32), ("d_model", _i32), ("d_inner", _i32),
        ("d_state", _i32), ("dt_rank", _i32), ("d_conv", _i32), ("fold", _i32), ("reserved", _i32),
    ]


# name -> (restype, argtypes); every symbol of include/mtl.h
SIGNATURES = {
    "mtl_last_error": (ctypes.c_char_p, []),
    "mtl_abi_version": (ctypes.c_int, []),
    "mtl_selective_scan_fwd": (ctypes.c_int, [ctypes.POINTER(ScanParams), _vp]),
    "mtl_causal_conv1d_fwd": (ctypes.c_int, [ctypes.POINTER(ConvParams), _vp]),
    "mtl_conv_step": (ctypes.c_int, [_vp, _vp, _i64, _fp, _fp, _vp, _i64, _i64, _i64, _i32, _i32, _i32, _vp]),
    "mtl_selective_state_update": (ctypes.c_int, [_fp, _vp, _i64, _vp, _i64, _vp, _i64, _fp, _fp, _fp, _fp,
                                                  _vp, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _vp]),
    "mtl_add_rmsnorm": (ctypes.c_int, [_fp, _fp, _fp, _fp, _fp, _i64, _i64, ctypes.c_float, _vp]),
    "mtl_add_rmsnorm_parts": (ctypes.c_int, [_fp, _fp, _i32, _fp, _fp, _fp, _i64, _i64, ctypes.c_float, _vp]),
    "mtl_sum_parts": (ctypes.c_int, [_fp, _i32, _i64, _fp, _vp]),
    "mtl_xproj_sum_dt": (ctypes.c_int, [_fp, _i32, _i64, _i32, _fp, _i32, _i64, _fp, _fp, _vp]),
    "mtl_prefill_short": (ctypes.c_int, [ctypes.POINTER(PrefillShortArgs), ctypes.POINTER(PrefillLayer), _vp]),
    "mtl_prefill_long": (ctypes.c_int, [ctypes.POINTER(PrefillLongArgs), ctypes.POINTER(PrefillLayer), _vp]),
    "mtl_decode_step": (ctypes.c_int, [ctypes.POINTER(DecodeStepArgs), ctypes.POINTER(DecodeLayer), _vp]),
    "mtl_decode_step_batched": (ctypes.c_int, [ctypes.POINTER(DecodeStepBatchedArgs), ctypes.POINTER(DecodeLayer),
                                               _vp]),
    "mtl_decode_persist_workspace_bytes": (ctypes.c_size_t, [_i32, _i32, _i32, _i32]),
    "mtl_decode_persist_grid": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "mtl_decode_step_persist": (ctypes.c_int, [ctypes.POINTER(DecodeStepArgs), ctypes.POINTER(DecodeLayer), _vp, _vp,
                                               ctypes.c_size_t, _i32, _vp]),
    "mtl_conv_step_xproj": (ctypes.c_int, [_fp, _fp, _i64, _fp, _fp, _fp, _i64, _fp, _fp, _i64, _i64, _i32, _i32,
                                           _vp]),
    "mtl_conv_step_xproj_noalloc": (ctypes.c_int, [_fp, _fp, _i64, _fp, _fp, _fp, _i64, _fp, _fp, _i64, _i64, _i32,
                                                   _i32, _vp]),
    "mtl_quant_dequant_sum_int8_tok": (ctypes.c_int, [ctypes.POINTER(_vp), _i32, _i64, _i64,
                                                      ctypes.POINTER(_vp), _fp, _vp]),
    "mtl_quant_dequant_sum_fp16": (ctypes.c_int, [ctypes.POINTER(_vp), _i32, _i64, ctypes.POINTER(_vp), _fp, _vp]),
    "mtl_decode_in": (ctypes.c_int, [_fp, _fp, _vp, _i32, _fp, _fp, ctypes.c_float, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp,
                                     _fp, _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "mtl_decode_gemv": (ctypes.c_int, [_fp, _fp, _fp, _fp, _fp, _i32, _i32, _i32, _vp]),
    "mtl_decode_gemv_parts": (ctypes.c_int, [_fp, _fp, _fp, _i32, _i32, _i32, _i32, _vp]),
    "mtl_linear_skinny": (ctypes.c_int, [_fp, _i64, _fp, _fp, _fp, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _vp]),
    "mtl_in_proj_conv_prefill": (ctypes.c_int, [_fp, _i64, _fp, _fp, _fp, _fp, _i32, _fp, _fp, _fp, _fp, _i64, _i64,
                                                _i64, _i64, _vp]),
    "mtl_in_proj_conv_xproj": (ctypes.c_int, [_fp, _i64, _fp, _fp, _fp, _fp, _fp, _i32, _fp, _i32, _fp, _fp, _i64, _fp,
                                              _i64, _i64, _i64, _i32, _vp]),
    "mtl_in_proj_conv_xproj_normed": (ctypes.c_int, [_fp, _i64, _fp, _fp, _fp, _fp, _fp, _i32, _fp, _i32, _fp, _fp,
                                                     _i64, _fp, _i64, _i64, _i64, _i32, _fp, _i32, ctypes.c_float,
                                                     _vp]),
    "mtl_linear_skinny_residual": (ctypes.c_int, [_fp, _i64, _fp, _fp, _fp, _i64, _i64, _i64, _i32, _i32, _fp, _fp,
                                                  _fp, _fp, _vp, _vp]),
    "mtl_decode_norm_gemv": (ctypes.c_int, [_fp, _fp, ctypes.c_float, _fp, _fp, _fp, _i32, _i32, _i32, _vp]),
    "mtl_decode_ssm": (ctypes.c_int, [_fp, _i32, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _i32, _i32, _i32, _i32,
                                      _vp]),
}

_lib = None


class MTLError(RuntimeError):
    """A libmtl entry point returned a nonzero status."""


def load() -> ctypes.CDLL:
    """Opens libmtl.so once and declares every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise MTLError(f"{LIB_PATH} is not built; run `python mamba-tp-lite_amd/build.py` "
                       "(or __graft_entry__.build()) first -- there is no CPU fallback")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.mtl_abi_version()
    if ver != ABI_VERSION:
        raise MTLError(f"libmtl ABI version {ver}, expected {ABI_VERSION}; rebuild the library")
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().mtl_last_error().decode(errors="replace")
        raise MTLError(f"{what} failed (status {status}): {msg}")
