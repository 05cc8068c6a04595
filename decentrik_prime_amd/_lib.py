"""ctypes binding of libdk.so, the C ABI declared in include/dk.h.

The library is loaded once (thread-safe) from this package directory.  There is no fallback: if
libdk.so is missing or a symbol is absent, every operator raises.  Arguments are raw device
pointers (``tensor.data_ptr()``) and the stream handle of ``torch.cuda.current_stream()``.
"""

import ctypes
import os
import re
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libdk.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "dk.h")

DK_ERR_INVALID = -1
DK_ERR_ALIGN = -2
DK_ERR_WORKSPACE = -3
DK_ERR_CAPTURE = -4
DK_OUT_F16, DK_OUT_F32, DK_OUT_F32_ACCUM = 0, 1, 2
DK_NOALLOC_SCRATCH_BYTES = 64 << 20
DK_OP_LINEAR_FWD, DK_OP_LINEAR_BWD_DX, DK_OP_GATEUP_SWIGLU_FWD, DK_OP_DOWN_SWIGLU_BWD = 0, 1, 2, 3
DK_W4_KERNEL_AUTO, DK_W4_KERNEL_TILE, DK_W4_KERNEL_STAGED = 0, 1, 2

_c_p, _i64, _int, _f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float


class NF4WeightC(ctypes.Structure):
    """struct dk_nf4_weight."""
    _fields_ = [("packed", _c_p), ("qabs", _c_p), ("scale2", _c_p), ("offset2", _c_p),
                ("code2", _c_p), ("nf4", _c_p), ("rows", _i64), ("cols", _i64),
                ("kernel", ctypes.c_int32)]


_W = ctypes.POINTER(NF4WeightC)


class LoraTermC(ctypes.Structure):
    """struct dk_lora_term."""
    _fields_ = [("left", _c_p), ("right", _c_p), ("mask", _c_p), ("col_begin", _i64),
                ("col_end", _i64), ("scale", _f32)]


_T = ctypes.POINTER(LoraTermC)


class LoraDownTermC(ctypes.Structure):
    """struct dk_lora_down_term."""
    _fields_ = [("mask", _c_p), ("keep_scale", _f32), ("a", _c_p), ("z", _c_p), ("x", _c_p)]


class LoraGradsTermC(ctypes.Structure):
    """struct dk_lora_grads_term."""
    _fields_ = [("dy", _c_p), ("lddy", _i64), ("n_out", _i64), ("z", _c_p), ("lora_b", _c_p),
                ("lora_scale", _f32), ("mask", _c_p), ("keep_scale", _f32), ("da", _c_p),
                ("db", _c_p), ("dz", _c_p), ("x", _c_p)]


class SideLoraSumsC(ctypes.Structure):
    """struct dk_side_lora_sums."""
    _fields_ = [("x", _c_p), ("m", _i64), ("k", _i64), ("rank", _i64),
                ("terms", ctypes.POINTER(LoraGradsTermC)), ("n_terms", ctypes.c_int32)]


class SideDequantC(ctypes.Structure):
    """struct dk_side_dequant."""
    _fields_ = [("packed", _c_p), ("qabs", _c_p), ("scale2", _c_p), ("offset2", _c_p),
                ("code2", _c_p), ("nf4", _c_p), ("out", _c_p), ("sb0", _i64), ("sb1", _i64),
                ("wgs", ctypes.c_int32)]


_S = ctypes.POINTER(SideDequantC)


class RopeC(ctypes.Structure):
    """struct dk_rope."""
    _fields_ = [("pos", _c_p), ("cos_table", _c_p), ("sin_table", _c_p), ("hd", ctypes.c_int32),
                ("cols", _i64)]

# name -> (restype, argtypes)
SIGNATURES = {
    "dk_error_string": (ctypes.c_char_p, [_int]),
    "dk_nf4_dequant": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _c_p]),
    "dk_nf4_quantize": (_int, [_c_p, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "dk_gated_silu_fwd": (_int, [_c_p, _c_p, _i64, _i64, _c_p]),
    "dk_gated_silu_bwd": (_int, [_c_p, _c_p, _i64, _i64, _c_p]),
    "dk_swiglu_fwd": (_int, [_c_p, _c_p, _c_p, _i64, _c_p]),
    "dk_swiglu_bwd": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _i64, _c_p]),
    "dk_lora_down": (_int, [_c_p, _c_p, _f32, _c_p, _c_p, _i64, _i64, _i64, _c_p]),
    "dk_w4_linear_fwd": (_int, [_c_p, _i64, _i64, _W, _c_p, _c_p, _c_p, _i64, _f32, _c_p, _i64,
                                _c_p, _i64, _c_p]),
    "dk_w4_linear_bwd_dx": (_int, [_c_p, _i64, _i64, _W, _c_p, _c_p, _i64, _c_p, _f32, _c_p,
                                   _i64, _int, _c_p, _i64, _c_p]),
    "dk_w4_linear_fwd_lora": (_int, [_c_p, _i64, _i64, _W, _c_p, _T, _int, _i64, _c_p, _i64,
                                     _c_p, _i64, _c_p]),
    "dk_w4_linear_bwd_dx_lora": (_int, [_c_p, _i64, _i64, _W, _T, _int, _i64, _c_p, _i64, _int,
                                        _c_p, _i64, _c_p]),
    "dk_w4_linear_workspace": (_i64, [_i64, _W, _int]),
    "dk_w4_workspace": (_i64, [_i64, _W, _int]),
    "dk_h16_workspace": (_i64, [_i64, _i64, _i64, _int]),
    "dk_h16_linear_fwd_lora": (_int, [_c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _T, _int, _i64,
                                      _c_p, _i64, _c_p, _i64, _S, _c_p]),
    "dk_h16_linear_fwd_rope": (_int, [_c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _T, _int, _i64,
                                      ctypes.POINTER(RopeC), _c_p, _i64, _S, _c_p]),
    "dk_h16_linear_bwd_dx_lora": (_int, [_c_p, _i64, _i64, _c_p, _i64, _i64, _T, _int, _i64, _c_p,
                                         _i64, _int, _c_p, _i64, _S, _c_p]),
    "dk_h16_linear_bwd_dx_lora_sums": (_int, [_c_p, _i64, _i64, _c_p, _i64, _i64, _T, _int, _i64,
                                              _c_p, _i64, _int, _c_p, _i64, _S,
                                              ctypes.POINTER(SideLoraSumsC), _c_p]),
    "dk_h16_linear_bwd_dx_lora_noalloc": (_int, [_c_p, _i64, _i64, _c_p, _i64, _i64, _T, _int,
                                                 _i64, _c_p, _i64, _int, _S, _c_p]),
    "dk_h16_gateup_swiglu_fwd": (_int, [_c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _c_p, _c_p, _i64,
                                        _S, _c_p]),
    "dk_h16_down_swiglu_bwd": (_int, [_c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _c_p, _i64, _S,
                                      _c_p]),
    "dk_lora_grads_workspace": (_i64, [_i64, _i64, _i64, _i64]),
    "dk_lora_down_multi": (_int, [_c_p, _i64, _i64, _i64, ctypes.POINTER(LoraDownTermC), _int, _c_p]),
    "dk_lora_down_multi_dequant": (_int, [_c_p, _i64, _i64, _i64, ctypes.POINTER(LoraDownTermC),
                                          _int, _S, _c_p]),
    "dk_lora_grads_multi_workspace": (_i64, [_i64, _i64, _i64, ctypes.POINTER(_i64), _int]),
    "dk_lora_grads_multi": (_int, [_c_p, _i64, _i64, _i64, ctypes.POINTER(LoraGradsTermC), _int,
                                   _c_p, _i64, _c_p]),
    "dk_lora_dz_multi": (_int, [_c_p, _i64, _i64, _i64, ctypes.POINTER(LoraGradsTermC), _int,
                                _c_p]),
    "dk_lora_grads": (_int, [_c_p, _i64, _c_p, _c_p, _c_p, _f32, _c_p, _f32, _i64, _i64, _i64,
                             _i64, _c_p, _c_p, _c_p, _c_p, _i64, _c_p]),
    "dk_rms_fwd": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _i64,
                          _f32, _f32, _c_p]),
    "dk_rms_bwd": (_int, [_c_p, _int, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                          _c_p, _c_p, _i64, _i64, _f32, _c_p]),
    "dk_qkv_epilogue_fwd": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _f32, _int, _int, _int,
                                   _c_p]),
    "dk_qkv_epilogue_bwd": (_int, [_c_p, _c_p, _c_p, _int, _c_p, _c_p, _c_p, _c_p, _i64, _int, _int,
                                   _int, _int, _c_p]),
    "dk_attn_fwd": (_int, [_c_p, _c_p, _int, _c_p, _int, _i64, _int, _int, _int, _c_p, _c_p, _c_p]),
    "dk_attn_bwd": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _int, _c_p, _int, _i64, _int, _int, _int,
                           _c_p, _c_p, _c_p, _c_p, _c_p]),
    "dk_head_chunk": (_int, [_c_p, _c_p, _c_p, _c_p, _i64, _i64, _i64, _i64, _f32, _i64, _c_p]),
    "dk_head_finalize": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _i64, _f32, _f32,
                                _i64, _c_p]),
    "dk_w4_gateup_swiglu_fwd": (_int, [_c_p, _i64, _i64, _W, _c_p, _c_p, _c_p, _i64, _c_p]),
    "dk_w4_down_swiglu_bwd": (_int, [_c_p, _i64, _i64, _W, _c_p, _c_p, _i64, _c_p]),
}

_lock = threading.Lock()
_lib = None


def header_symbols(path=HEADER):
    """Function names declared in include/dk.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dk_[a-z0-9_]+)\s*\(", text)))


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(f"{LIB_PATH} is not built: run `python -m decentrik_prime_amd.build`")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def check(rc, what):
    """Map a C-ABI return code to an exception: argument errors -> ValueError, launch errors ->
    RuntimeError."""
    if rc == 0:
        return
    msg = lib().dk_error_string(rc).decode()
    if rc < 0:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: HIP error {rc}: {msg}")


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(device=None):
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
