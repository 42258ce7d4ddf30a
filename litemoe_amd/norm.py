"""Decode RMSNorm on the gfx950 kernel; keeps the reference's bf16 rounding
before the weight multiply (litemoe/norm.py:7-29, model.py:9-11)."""
import torch

from . import _lib


def _validate(x, weight):
    if not x.is_cuda or not x.is_contiguous() or not weight.is_contiguous():
        raise ValueError('Fused RMSNorm requires contiguous CUDA tensors')
    if weight.ndim != 1 or weight.numel() != x.shape[-1] or weight.dtype != x.dtype or weight.device != x.device:
        raise ValueError('Fused RMSNorm weight must match the last dimension, dtype and device')
    if x.dtype != torch.bfloat16:
        raise ValueError('Fused RMSNorm supports BF16')


def rmsnorm(x, weight, eps, out=None):
    """``bf16(x * rsqrt(mean(x^2) + eps)) * weight`` (norm.py:19-29)."""
    _validate(x, weight)
    out = torch.empty_like(x) if out is None else out
    width = x.shape[-1]
    if x.numel():
        _lib.call("lm_rmsnorm", x.data_ptr(), weight.data_ptr(), out.data_ptr(),
                  x.numel() // width, width, float(eps), _lib.stream(x.device))
    return out


def add_rmsnorm(x, a, alpha, weight, eps, out=None):
    """In place ``x <- bf16(x + alpha * a)`` then ``rmsnorm(x)``.

    Fuses the residual update ``x.add(a, alpha=residual_multiplier)`` with the
    following norm (litemoe/model.py:108-109, :122 with the next layer's :106).
    """
    _validate(x, weight)
    if a is not None and (a.shape != x.shape or a.dtype != x.dtype or not a.is_contiguous() or not a.is_cuda):
        raise ValueError('Residual input must match x and be contiguous')
    out = torch.empty_like(x) if out is None else out
    width = x.shape[-1]
    if x.numel():
        _lib.call("lm_add_rmsnorm", x.data_ptr(), _lib.ptr(a), float(alpha), weight.data_ptr(),
                  out.data_ptr(), x.numel() // width, width, float(eps), _lib.stream(x.device))
    return out
