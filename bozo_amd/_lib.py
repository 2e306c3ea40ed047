"""ctypes binding of libtension_hip.so (the C ABI declared in include/tension_hip.h).

torch is imported first on purpose: torch ships its own libamdhip64 whose
SONAME (libamdhip64.so.7) is the one libtension_hip.so needs, so the library
binds to the HIP runtime torch already loaded and torch's stream handles and
device pointers are valid inside it.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libtension_hip.so")

# dtype codes (enum in tension_hip.h)
F32, BF16, F16, F64 = 0, 1, 2, 3
DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.float64: F64}

# flags
NORM_MASS = 1 << 0
NORM_COUNT = 1 << 1
GLOBAL = 1 << 2
FORCE_EXACT = 1 << 3
DECODE_SELF = 1 << 4
TAU_VALID_ONLY = 1 << 5

# bytes of the fixed device scratch of tension_global_bwd_noalloc
NOALLOC_SCRATCH_BYTES = 8 << 20

# kernel families (tension_last_kernel)
KERNEL_EXACT, KERNEL_MFMA, KERNEL_SPLIT_BF16, KERNEL_SPLIT_F32, KERNEL_SPLIT_F32V, KERNEL_SPLIT_F16 = 0, 1, 2, 3, 4, 5

# status codes
OK, ERR_ARG, ERR_UNSUPPORTED, ERR_LAUNCH = 0, 1, 2, 3
_STATUS = {ERR_ARG: "bad argument", ERR_UNSUPPORTED: "unsupported", ERR_LAUNCH: "launch failure"}


class TensionBuf(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("dtype", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("s", ctypes.c_int64 * 4)]


BufP = ctypes.POINTER(TensionBuf)
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f64 = ctypes.c_double
_vp = ctypes.c_void_p

# name -> (restype, argtypes)
SIGNATURES = {
    "tension_window_fwd": (_i32, [BufP] * 7 + [_i64] * 5 + [_f64, _i32, _vp]),
    "tension_window_bwd_workspace": (_i64, [_i64, _i64, _i64, _i32, _i32]),
    "tension_window_bwd": (_i32, [BufP] * 9 + [_vp] + [_i64] * 5 + [_f64, _i32, _vp]),
    "tension_window_bwd_saved": (_i32, [BufP] * 11 + [_vp] + [_i64] * 5 + [_f64, _i32, _vp]),
    "tension_window_bwd_dq": (_i32, [BufP] * 7 + [_vp] + [_i64] * 5 + [_f64, _i32, _vp]),
    "tension_window_bwd_dkv": (_i32, [BufP] * 8 + [_vp] + [_i64] * 5 + [_f64, _i32, _vp]),
    "tension_global_fwd": (_i32, [BufP] * 7 + [_i64] * 5 + [_f64, _i32, _vp]),
    "tension_global_bwd_workspace": (_i64, [_i64, _i64, _i64, _i32, _i32]),
    "tension_global_bwd": (_i32, [BufP] * 11 + [_vp] + [_i64] * 5 + [_f64, _i32, _vp]),
    "tension_global_bwd_noalloc": (_i32, [BufP] * 11 + [_i64] * 5 + [_f64, _i32, _vp]),
    "tension_decode_step": (_i32, [BufP] * 7 + [_vp, _vp] + [_i64] * 4 + [_f64, _i32, _vp]),
    "tension_rope": (_i32, [BufP, BufP, _vp, _vp] + [_i64] * 6 + [_i32, _vp]),
    "tension_tau_head_stats": (_i32, [BufP, _i32] + [_i64] * 4 + [_vp, _i32, _vp]),
    "tension_tau_aggregate": (_i32, [BufP, _i32] + [_i64] * 4 + [_vp, _vp, _vp]),
    "tension_bias_table_insert": (_i32, [_vp, _vp, _i64, _vp, _vp, _i32, _vp]),
    "tension_aux_loss_partials": (_i64, [_i64, _i64, _i64]),
    "tension_aux_loss_fwd": (_i32, [BufP, _i32] + [_i64] * 4 + [_vp, _vp]),
    "tension_aux_loss_bwd": (_i32, [BufP, BufP, _i32] + [_i64] * 4 + [_vp, _vp]),
    "tension_bias_build": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _i32, _f64, BufP, _vp, _vp]),
    "tension_last_error": (ctypes.c_char_p, []),
    "tension_version": (ctypes.c_char_p, []),
    "tension_last_kernel": (_i32, []),
}

_lib = None


class TensionError(RuntimeError):
    pass


def lib():
    """Load (once) and return the library; raise if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise TensionError(
                f"{LIB_PATH} is missing: build it with `python -m bozo_amd.build` "
                "(there is no CPU fallback for the tension kernels)")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def check(status: int, what: str) -> None:
    if status != OK:
        msg = lib().tension_last_error().decode(errors="replace")
        raise TensionError(f"{what}: {_STATUS.get(status, status)}: {msg}")


def buf(t: torch.Tensor | None):
    """TensionBuf pointer for a tensor (None -> NULL).  Strides are in
    elements, padded with zeros to 4 entries."""
    if t is None:
        return None
    code = DTYPE_CODE.get(t.dtype)
    if code is None:
        raise TypeError(f"unsupported dtype {t.dtype}")
    if t.dim() > 4:
        raise ValueError(f"a tension_buf describes at most 4 dimensions, got {t.dim()}")
    s = list(t.stride()) + [0] * (4 - t.dim())
    b = TensionBuf(ctypes.c_void_p(t.data_ptr()), code, 0, (ctypes.c_int64 * 4)(*s[:4]))
    return ctypes.pointer(b)


def stream_handle(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream
