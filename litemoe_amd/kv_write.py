"""Conflict-free masked KV stores on the gfx950 kernel (litemoe/kv_write.py)."""
import torch

from . import _lib


def write(cache, layer, k, v, positions, active, slots):
    """Store ``k[row, h, 0, c]`` at ``cache.k[layer, slots[row], h, positions[row], c]``
    for active rows (same for v). Inputs may have strided heads/channels; the
    cache is contiguous ``[B, H, C, D]`` (kv_write.py:23-29, index :16)."""
    _, heads, _, dim = k.shape
    kc, vc = cache.k[layer], cache.v[layer]
    _lib.require_cuda(k, v, kc, vc, what="KV write tensors")
    if k.dtype != kc.dtype or v.dtype != vc.dtype or kc.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError('KV write requires matching BF16 or FP32 tensors')
    if not kc.is_contiguous() or not vc.is_contiguous():
        raise ValueError('KV cache layers must be contiguous')
    rows = k.shape[0]
    positions = positions.to(torch.int64).contiguous()
    active = active.to(torch.bool).contiguous()
    slots = slots.to(torch.int64).contiguous()
    if positions.numel() != rows or active.numel() != rows or slots.numel() != rows:
        raise ValueError('positions, active and slots need one entry per row')
    _lib.call("lm_kv_write", k.data_ptr(), k.stride(0), k.stride(1), k.stride(3),
              v.data_ptr(), v.stride(0), v.stride(1), v.stride(3), kc.data_ptr(), vc.data_ptr(),
              positions.data_ptr(), active.data_ptr(), slots.data_ptr(), rows, heads, dim,
              cache.capacity, kc.shape[0], kc.element_size(), _lib.stream(kc.device))
