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


class Plan(ctypes.Structure):
    """mi_fa2_plan: how the launches are sized for a device (its CUs and XCDs)."""
    _fields_ = [("num_cus", ctypes.c_int32), ("num_xcds", ctypes.c_int32),
                ("xcds_mapped", ctypes.c_int32), ("decode_work_groups_paged", ctypes.c_int32),
                ("decode_work_groups_dense", ctypes.c_int32),
                ("prefill_one_stream_min_work_groups", ctypes.c_int32),
                ("prefill_one_stream_max_keys", ctypes.c_int32)]


# name -> (restype, argtypes); mirrors include/mi_fa2.h
SIGNATURES = {
    "mi_fa2_version": (ctypes.c_char_p, []),
    "mi_fa2_last_error": (ctypes.c_char_p, []),
    "mi_fa2_launch_plan": (_i32, [_i32, _i32, ctypes.POINTER(Plan)]),
    "mi_fa2_set_clock_probe": (_i32, [_p]),
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


def device_index(dev):
    """The index of a cuda device ("cuda" alone: the current one)."""
    return dev.index if dev.index is not None else torch._C._cuda_getDevice()


class on_device:
    """`with on_device(dev) as stream:` makes dev the current device for the block (only if it is
    not already: the common case costs two integer reads) and yields the raw handle of dev's
    current stream, the stream a launch goes to."""
    __slots__ = ("idx", "prev")

    def __init__(self, dev):
        self.idx = device_index(dev)

    def __enter__(self):
        self.prev = torch._C._cuda_getDevice()
        if self.prev != self.idx:
            torch._C._cuda_setDevice(self.idx)
        return torch._C._cuda_getCurrentRawStream(self.idx)

    def __exit__(self, *exc):
        if self.prev != self.idx:
            torch._C._cuda_setDevice(self.prev)
        return False


def launch_plan(num_cus=0, num_xcds=0):
    """The launch plan for a device of num_cus CUs in num_xcds XCDs, or (num_cus <= 0) for the
    current device."""
    pl = Plan()
    check(load().mi_fa2_launch_plan(num_cus, num_xcds, ctypes.byref(pl)))
    return {name: getattr(pl, name) for name, _ in Plan._fields_}
