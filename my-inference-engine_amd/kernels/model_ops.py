"""Fused residual add + RMSNorm and SwiGLU on the HIP kernels (csrc/model_ops.hip).

`add_rmsnorm(x, weight, eps, y=None)` replaces the reference's residual add (model.py:128-138)
followed by RMSNorm (model.py:49-55, eight torch ops), `silu_mul(gate_up)` replaces
F.silu(gate) * up (model.py:112-120), each as one launch with the reference's rounding points.
No CPU path: CPU tensors are rejected.
"""
import torch

from . import _lib


def _rows(t, name):
    assert t.is_cuda and t.dtype in _lib.DTYPES, f"{name}: a bf16 / fp16 GPU tensor"
    assert t.dim() == 2 and t.stride(1) == 1, f"{name}: [rows, n] with unit column stride"
    return t


def add_rmsnorm(x, weight, eps, y=None, residual_out=None, out=None):
    """x [rows, hidden] (+ y) -> (r, out): r = x + y rounded (x itself when y is None), out =
    weight * rmsnorm(r).  residual_out may be x (in place).  Returns (r, out)."""
    _rows(x, "x")
    R, H = x.shape
    if y is not None:
        _rows(y, "y")
        assert y.shape == x.shape and y.dtype == x.dtype
        if residual_out is None:
            residual_out = torch.empty_like(x)
        _rows(residual_out, "residual_out")
    if out is None:
        out = torch.empty((R, H), device=x.device, dtype=x.dtype)
    _rows(out, "out")
    assert weight.is_cuda and weight.dtype == x.dtype and weight.shape == (H,) and weight.is_contiguous()
    lib = _lib.load()
    _lib.check(lib.mi_fa2_add_rmsnorm(
        _lib.DTYPES[x.dtype], x.data_ptr(), x.stride(0) if R > 1 else H,
        y.data_ptr() if y is not None else None, (y.stride(0) if R > 1 else H) if y is not None else 0,
        weight.data_ptr(), residual_out.data_ptr() if y is not None else None,
        (residual_out.stride(0) if R > 1 else H) if y is not None else 0, out.data_ptr(),
        out.stride(0) if R > 1 else H, R, H, float(eps), _lib.stream_of(x)))
    return (residual_out if y is not None else x), out


def silu_mul(gate_up, out=None):
    """gate_up [rows, 2 * inter] (gate first) -> silu(gate) * up [rows, inter]."""
    _rows(gate_up, "gate_up")
    R, I2 = gate_up.shape
    assert I2 % 2 == 0
    inter = I2 // 2
    if out is None:
        out = torch.empty((R, inter), device=gate_up.device, dtype=gate_up.dtype)
    _rows(out, "out")
    lib = _lib.load()
    _lib.check(lib.mi_fa2_silu_mul(
        _lib.DTYPES[gate_up.dtype], gate_up.data_ptr(), gate_up.stride(0) if R > 1 else I2,
        out.data_ptr(), out.stride(0) if R > 1 else inter, R, inter, _lib.stream_of(gate_up)))
    return out
