# SPDX-License-Identifier: Apache-2.0
"""ctypes binding of libexl3_mi355x.so (the C ABI declared in include/exl3_mi355x.h).

torch is imported before the library is opened: the library's libamdhip64.so.7 dependency then binds to
the HIP runtime torch already loaded (same SONAME), so kernels, device pointers and stream handles all
belong to one runtime. There is no fallback: if the library is missing or fails to load, every entry
point raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede loading the library, see above)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libexl3_mi355x.so")

_c_int, _c_uint, _c_size, _c_float, _vp = ctypes.c_int, ctypes.c_uint, ctypes.c_size_t, ctypes.c_float, ctypes.c_void_p

_SIGNATURES = {
    "exl3_version": (_c_int, []),
    "exl3_last_error": (ctypes.c_char_p, []),
    "exl3_codebook": (_c_int, [_c_int, _c_int, _vp, _vp]),
    "exl3_reconstruct": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp]),
    "exl3_gemv_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "exl3_gemv": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _c_int, _c_uint,
                           _vp, _c_size, _vp]),
    "exl3_gemv_ex": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _c_int, _c_uint,
                              _vp, _c_size, _c_int, _vp]),
    "exl3_gemv_noalloc": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _c_int,
                                   _c_uint, _vp]),
    "exl3_gemv_fused": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _c_float, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int,
                                 _c_int, _vp, _vp, _vp, _c_int, _c_int, _c_uint, _vp, _vp, _vp, _c_size, _vp]),
    "exl3_gemv_fused_mk": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _c_float, _vp, _vp, _vp, _c_int, _vp, _vp,
                                    _c_int, _c_int, _vp, _vp, _vp, _c_int, _c_int, _c_uint, _vp, _vp, _vp, _c_size,
                                    _vp]),
    "exl3_rotate": (_c_int, [_vp, _c_int, _vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "exl3_rmsnorm_rotate": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_float, _vp, _c_int, _c_int, _c_int, _vp, _vp,
                                     _vp]),
    "exl3_swiglu_rotate": (_c_int, [_vp, _vp, _c_int, _c_int, _vp, _vp]),
    "exl3_prefill_gemm": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _c_int, _vp]),
    "exl3_prefill_matmul": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _c_int, _vp, _c_size,
                                     _vp]),
    "exl3_prefill_matmul_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "exl3_prefill_out_rotate": (_c_int, [_vp, _c_int, _c_int, _vp, _vp, _vp, _c_int, _vp]),
    "exl3_attn_decode_rotate": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp,
                                         _vp, _vp, _vp]),
}

EXPORTED = tuple(_SIGNATURES)

_lib = None


class Exl3Error(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise Exl3Error(f"{LIB_PATH} is not built: run `python omlx-exl3_amd/build.py` "
                            "(or __graft_entry__.build())")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().exl3_last_error().decode(errors="replace")
        raise Exl3Error(f"{what} failed ({rc}): {msg}")


def stream_handle(device: torch.device | None = None) -> int:
    """The current torch stream of `device` as a raw hipStream_t."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


DTYPE_CODE = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
