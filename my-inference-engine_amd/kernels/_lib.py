"""ctypes binding of libmi_fa2.so (the C ABI declared in include/mi_fa2.h).

The library is built in-tree by build_lib.py next to this file.  It links libamdhip64.so.7, the
same SONAME as the HIP runtime bundled with PyTorch-ROCm, so once torch is imported the loader
reuses torch's runtime and the kernels run on torch's streams and allocations.

There is no fallback: if the library is missing or fails to load, every call raises.
"""
import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must be loaded first: provides the HIP runtime the library binds to)

LIB_PATH = Path(os.environ.get("MI_FA2_LIB", Path(__file__).resolve().parent / "libmi_fa2.so"))

OK = 0
DTYPES = {torch.bfloat16: 0, torch.float16: 1}
GENERAL_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}  # mi_fa2_fwd_general

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/mi_fa2.h
SIGNATURES = {
    "mi_fa2_version": (ctypes.c_char_p, []),
    "mi_fa2_last_error": (ctypes.c_char_p, []),
    "mi_fa2_fwd_workspace_size": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "mi_fa2_fwd": (_i32, [_i32, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32,
                          _p, _p, _p, _p, _p, _i32, _f32, _p, _sz, _p]),
    "mi_fa2_fwd_general": (_i32, [_i32, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32,
                                  _i32, _i32, _p, _p, _p, _p, _p, _i32, _f32, _p]),
    "mi_fa2_fwd_varlen": (_i32, [_i32, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32,
                                 _p, _p, _p, _p, _p, _i32, _f32, _p]),
    "mi_fa2_fwd_paged_workspace_size": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "mi_fa2_rope_kv_write": (_i32, [_i32, _p, _i64, _p, _p, _i64, _p, _i32, _i32, _i32, _i32, _p,
                                    _i64, _p, _p, _p, _i32, _p]),
    "mi_fa2_fwd_paged": (_i32, [_i32, _p, _p, _p, _p, _p, _p, _i64, _p, _i32, _i32, _i32, _i32,
                                _i32, _i32, _i32, _i32, _p, _p, _p, _p, _i32, _f32, _p, _sz, _p]),
    "mi_fa2_fwd_paged_noalloc": (_i32, [_i32, _p, _p, _p, _p, _p, _p, _i64, _p, _i32, _i32, _i32,
                                        _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _i32, _f32,
                                        _p]),
    "mi_fa2_step_metadata": (_i32, [_p, _p, _i32, _i32, _p, _i32, _p, _i64, _i32, _i32, _p, _p,
                                    _p, _p, _p, _p, _p]),
    "mi_fa2_add_rmsnorm": (_i32, [_i32, _p, _i64, _p, _i64, _p, _p, _i64, _p, _i64, _i32, _i32,
                                  _f32, _p]),
    "mi_fa2_silu_mul": (_i32, [_i32, _p, _i64, _p, _i64, _i32, _i32, _p]),
    "mi_fa2_sample_workspace_size": (_sz, [_i32, _i32]),
    "mi_fa2_sample": (_i32, [_i32, _p, _i64, _i32, _i32, _f32, ctypes.c_uint64, ctypes.c_uint64,
                             _p, _p, _sz, _p]),
    "mi_fa2_combine": (_i32, [_i32, _p, _p, _p, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p,
                              _p]),
    "mi_fa2_fwd_paged_varlen": (_i32, [_i32, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i32, _i32,
                                       _i32, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _i32,
                                       _f32, _p]),
}

_lib = None


class MiFa2Error(RuntimeError):
    """A libmi_fa2 entry point returned a non-zero status."""


def load():
    """Load libmi_fa2.so once; raise if it is missing (there is no non-HIP path)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} not found: build it with `python my-inference-engine_amd/build_lib.py`"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status):
    if status != OK:
        msg = load().mi_fa2_last_error().decode()
        raise MiFa2Error(f"libmi_fa2 status {status}: {msg}")


def strides(t, n=None):
    """int64[n] array of t's strides (elements)."""
    s = t.stride()
    if n is not None:
        s = s[:n]
    return (ctypes.c_int64 * len(s))(*s)


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)
