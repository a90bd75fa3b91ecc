"""ctypes binding of libtjk.so (the C-ABI declared in include/tjk.h).

The library is built in-tree (``make -C tiktok-techjam-2026_amd/csrc`` or
``__graft_entry__.build()``) and loaded after ``import torch`` so that it
shares torch's HIP runtime (both link ``libamdhip64.so.7``): the stream
handles torch hands out are then valid inside the library.  There is no
fallback: if the library is missing, every op raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede the library load; see module docstring)

LIB_PATH = Path(__file__).with_name("libtjk.so")
ABI_VERSION = 10

F32, F16, BF16 = 0, 1, 2
OK, EINVAL, EUNSUPPORTED = 0, -1, -2
EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_RESIDUAL = 0, 1, 2

DTYPE_CODES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_lib = None

_vp, _i64, _i32, _f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float

_SIGNATURES = {
    "tjk_abi_version": (_i32, []),
    "tjk_last_error_string": (ctypes.c_char_p, []),
    "tjk_add_layernorm": (_i32, [_vp, _i32, _i64, _vp, _i32, _i64, _i32, _i64, _vp, _i32, _i64, _vp, _i32, _i64,
                                 _vp, _vp, _i64, _i64, _f32, _vp, _i64, _vp, _vp, _vp]),
    "tjk_gemm_bias": (_i32, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64,
                             _i32, _i32, _i32, _vp]),
    "tjk_gemm_bias_residual_from": (_i32, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64,
                                           _vp, _i64, _i64, _vp, _vp, _i32, _i32, _vp]),
    "tjk_gemm_plan_count": (_i32, [_i32]),
    "tjk_gemm_plan_info": (_i32, [_i32, _i32, ctypes.POINTER(_i32), ctypes.POINTER(_i32),
                                  ctypes.POINTER(_i32), ctypes.POINTER(_i32)]),
    "tjk_flash_fwd": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _i32, _i32, _i32, _i32,
                             _f32, _i32, _vp, _vp, _vp, _i32, _i32, _vp]),
    "tjk_flash_plan_count": (_i32, [_i32]),
    "tjk_flash_fwd_sched": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _f32, _i32,
                                   _vp, _vp, _i32, _i32, _vp, ctypes.c_size_t, _i32, _i32, _vp]),
    "tjk_flash_partial_bytes": (ctypes.c_size_t, [_i32, _i32]),
    "tjk_flash_fwd_sched_static": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _f32, _i32,
                                          _vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    "tjk_flash_sched_static_bytes": (ctypes.c_size_t, []),
    "tjk_flash_sched_occupancy": (_i32, [_i32, _i32]),
    "tjk_ffn": (_i32, [_vp, _i32, _i64, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32,
                       _i64, _i64, _i64, _i32, _vp]),
    "tjk_ffn_supported": (_i32, [_i64, _i64, _i32, _i32]),
    "tjk_attn_block": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _vp, _i32, _i32, _i32,
                              _i32, _f32, _i32, _i32, _vp]),
    "tjk_attn_block_supported": (_i32, [_i64, _i32, _i32, _i64, _i32]),
    "tjk_gemm_ln": (_i32, [_vp, _i64, _vp, _vp, _f32, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32,
                           _i32, _vp]),
    "tjk_gemm_ln_supported": (_i32, [_i64, _i32]),
    "tjk_gemm_ln_plan_count": (_i32, []),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


class TjkError(RuntimeError):
    """A tjk C-ABI call returned a non-zero status."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise TjkError(
            f"{LIB_PATH} is not built: run `make -C {LIB_PATH.parent.parent / 'csrc'}` "
            "or __graft_entry__.build(); tjkernels has no non-HIP fallback"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.tjk_abi_version()
    if version != ABI_VERSION:
        raise TjkError(f"libtjk ABI version {version}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().tjk_last_error_string().decode(errors="replace")
        raise TjkError(f"{what} failed with status {status}: {msg}")
