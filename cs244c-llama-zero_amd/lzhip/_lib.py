"""ctypes binding of libllamazero_hip.so (declared in include/llamazero_hip.h).

The library is loaded after torch so that the process keeps a single HIP
runtime (torch ships its own libamdhip64.so.7, which the dynamic loader then
reuses for this library).  There is no other compute path: if the library or a
GPU is missing, every op raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported before the HIP library is loaded)

LIB_NAME = "libllamazero_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

F32 = 0
BF16 = 1
F16 = 2

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_u64 = ctypes.c_uint64

# name -> (restype, argtypes); the order of arguments follows the header.
SIGNATURES = {
    "lz_last_error": (ctypes.c_char_p, []),
    "lz_version": (_i32, []),
    "lz_device_cus": (_i32, []),
    "lz_adamw": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i64, _f64, _f64, _f64, _f64, _f64, _i64, _vp, _vp]),
    "lz_adamw_step": (_i32, [_vp, _f64, _f64, _f64, _f64, _vp, _vp]),
    "lz_adamw_dev": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i64, _f64, _f64, _f64, _f64, _vp, _vp, _vp]),
    "lz_sumsq": (_i32, [_vp, _i32, _i64, _vp, _vp]),
    "lz_adamw_norm_workspace": (_i64, [_i64]),
    "lz_adamw_norm": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i64, _f64, _f64, _f64, _f64, _f64, _i64, _vp, _vp,
                             _vp, _i64, _vp]),
    "lz_adamw_multi": (_i32, [_vp, _i32, _i32, _i32, _f64, _f64, _f64, _f64, _f64, _i64, _vp, _vp, _vp]),
    "lz_sumsq_multi": (_i32, [_vp, _i32, _i32, _vp, _vp]),
    "lz_clip_finalize": (_i32, [_vp, _f32, _f32, _vp, _vp, _vp]),
    "lz_mt_gather": (_i32, [_vp, _i32, _i32, _vp, _i32, _i64, _i64, _i32, _vp]),
    "lz_mt_scatter": (_i32, [_vp, _i32, _vp, _i32, _i32, _i64, _i64, _vp]),
    "lz_mt_gather_host": (_i32, [_vp, _i32, _i32, _vp, _i32, _i64, _i64, _i32, _vp]),
    "lz_mt_scatter_host": (_i32, [_vp, _i32, _vp, _i32, _i32, _i64, _i64, _vp]),
    "lz_axpy_f32": (_i32, [_vp, _vp, _i32, _i64, _f32, _vp]),
    "lz_add_inplace": (_i32, [_vp, _vp, _i32, _i64, _vp]),
    "lz_scale_inplace": (_i32, [_vp, _i32, _i64, _f32, _vp]),
    "lz_scale_dev": (_i32, [_vp, _i32, _i64, _vp, _vp]),
    "lz_fill": (_i32, [_vp, _i32, _i64, _f64, _vp]),
    "lz_cast": (_i32, [_vp, _i32, _vp, _i32, _i64, _vp]),
    "lz_rmsnorm_fwd": (_i32, [_vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _f32, _vp]),
    "lz_rmsnorm_bwd_workspace": (_i64, [_i64, _i64]),
    "lz_rmsnorm_bwd": (
        _i32,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _i64, _i32, _i64, _i64, _i64, _i64, _i64, _vp],
    ),
    "lz_rmsnorm_bwd_noalloc": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _vp]),
    "lz_rope_table": (_i32, [_vp, _vp, _i32, _i64, _i64, _vp, _i32, _vp]),
    "lz_rope": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _i32, _vp]),
    "lz_swiglu_fwd": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i32, _vp]),
    "lz_swiglu_bwd": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i32, _vp]),
    "lz_embedding_fwd": (_i32, [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _i32, _vp, _vp]),
    "lz_embedding_bwd": (_i32, [_vp, _i64, _vp, _i64, _i64, _i64, _vp, _i32, _vp, _i32, _vp]),
    "lz_ce_fwd": (_i32, [_vp, _i64, _i64, _i64, _i32, _vp, _i64, _i64, _vp, _vp, _vp]),
    "lz_ce_reduce": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _i32, _vp]),
    "lz_ce_bwd": (_i32, [_vp, _i64, _i64, _i64, _i32, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i32, _vp]),
    "lz_transpose": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp]),
    "lz_copy2d": (_i32, [_vp, _i64, _vp, _i64, _i64, _i64, _i32, _vp]),
    "lz_gemm_nt": (_i32, [_vp, _i64, _vp, _i64, _i32, _vp, _i64, _i32, _vp, _i64, _i64, _i64, _i64, _f32, _f32, _vp]),
    "lz_gemm_swiglu": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp]),
    "lz_gemm_rope": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp]),
    "lz_gemm_rope_hd": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp]),
    "lz_gemm_swiglu_bwd": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp]),
    "lz_gemm": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _i32, _vp, _i64, _i32, _vp, _i64, _i64, _i64, _i64, _f32, _f32,
                       _vp, _i64, _vp]),
    "lz_gemm_f32": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _i64, _i32, _vp, _i64, _i64, _i64, _i64, _f32,
                           _f32, _vp, _i64, _vp]),
    "lz_gemm_f32_workspace": (_i64, [_i64, _i64, _i64]),
    "lz_gemm_f32_plan": (_i32, [_i64, _i64, _i64]),
    "lz_gemm_workspace": (_i64, [_i64, _i64, _i64, _i32, _i32]),
    "lz_gemm_plan": (_i32, [_i64, _i64, _i64, _i32, _i32]),
    "lz_attn_path": (_i32, [_i32, _i64, _i64, _i64, _i64, _i64, _i64]),
    "lz_attn_fwd": (
        _i32,
        [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _vp],
    ),
    "lz_attn_delta": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i32, _vp]),
    "lz_attn_fwd_general": (
        _i32,
        [
            _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i32, _vp, _f32, _u64, _vp, _i64, _vp, _i64, _i64, _i64, _i64,
            _i64, _f32, _i32, _vp,
        ],
    ),
    "lz_attn_bwd_general": (
        _i32,
        [
            _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i32, _vp, _f32, _u64, _vp, _i64, _vp, _i64,
            _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _vp,
        ],
    ),
    "lz_attn_bwd_with_o": (
        _i32,
        [
            _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _i64,
            _i64, _i64, _i64, _i64, _i64, _f32, _vp, _vp, _i32, _vp,
        ],
    ),
    "lz_dropout": (_i32, [_vp, _vp, _i64, _f32, _u64, _i32, _vp]),
    "lz_dropout_mask": (_i32, [_vp, _i64, _f32, _u64, _vp]),
    "lz_attn_bwd": (
        _i32,
        [
            _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _vp,
            _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _vp, _vp, _i32, _vp,
        ],
    ),
}

_lock = threading.Lock()
_lib = None


class HipLibraryError(RuntimeError):
    pass


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Loads (once) and returns the library with its signatures applied."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = Path(path) if path is not None else Path(os.environ.get("LLAMAZERO_HIP_LIB", LIB_PATH))
        if not p.exists():
            raise HipLibraryError(
                f"{p} is missing: build it with `python cs244c-llama-zero_amd/csrc/build.py` "
                "(the HIP kernels are the only compute path)"
            )
        lib = ctypes.CDLL(str(p), mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().lz_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise HipLibraryError(f"{what} failed ({rc}): {last_error()}")


def call(name: str, *args) -> None:
    """Calls an int-returning entry point and raises on a non-zero status."""
    fn = getattr(load(), name)
    check(fn(*args), name)
