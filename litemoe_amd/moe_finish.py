"""Weighted route reduction on the gfx950 kernel (litemoe/moe_finish.py)."""
import torch

from . import _lib


def finish(y, ids, order, scales, out, rank, count, logical=None):
    """FP32 ordered accumulation of rounded BF16 route contributions.

    ``y`` rows are in ``order`` (expert-sorted) position; for token t the
    routes are summed in ascending ``logical[ids]*K + j`` order, each term
    ``bf16(bf16(y) * bf16(scale))``. Non-local rows are never read.
    Validation and messages follow moe_finish.py:40-52.
    """
    tensors = (y, ids, order, scales, out)
    if any(not t.is_cuda or not t.is_contiguous() or t.device != y.device for t in tensors):
        raise ValueError('Fused combine requires contiguous tensors on one CUDA device')
    if ids.ndim != 2 or y.ndim != 2 or scales.shape != ids.shape:
        raise ValueError('Invalid route tensor shapes')
    batch, topk = ids.shape
    if y.shape[0] != ids.numel() or order.shape != (ids.numel(),) or out.shape != (batch, y.shape[1]):
        raise ValueError('Invalid route/output sizes')
    if y.dtype != torch.bfloat16 or out.dtype != y.dtype or not 0 < topk <= 8 or count <= 0:
        raise ValueError('Fused combine supports BF16 and top-k 1 through 8')
    remap = logical is not None and logical.numel() != 0
    if remap and (not logical.is_cuda or logical.device != y.device or not logical.is_contiguous()):
        raise ValueError('Logical map must be contiguous on the route device')
    ids32 = ids.to(torch.int32).contiguous()
    order64 = order.to(torch.int64).contiguous()
    scales32 = scales.to(torch.float32).contiguous()
    logical64 = logical.to(torch.int64).contiguous() if remap else None
    workspace = torch.empty(max(ids.numel(), 1), dtype=torch.int32, device=y.device)
    _lib.call("lm_moe_finish", y.data_ptr(), ids32.data_ptr(), order64.data_ptr(), scales32.data_ptr(),
              _lib.ptr(logical64), out.data_ptr(), batch, y.shape[1], topk, rank, count,
              workspace.data_ptr(), workspace.numel() * 4, _lib.stream(y.device))
    return out
