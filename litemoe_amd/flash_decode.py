"""Graph-safe split-K decode attention over each row's contiguous KV sequence.

Mirrors ``FlashDecode`` of litemoe/flash_decode.py:5-34: built once per
(batch, kv_heads, groups, capacity), called with ``q [B, Hq, 1, D]`` and the
layer caches ``k, v [B, Hkv, C, D]``; row b attends keys ``j < used[b]``
(``used = where(active, lengths + 1, 1)`` unless given). The split count is
fixed at construction, so the launch is capturable.

``fused_qkv`` is the decode layer's form: it takes the packed QKV
projection as split-K partials and applies the reduction, RoPE and the
KV-cache store of the new token itself (``lm_flash_decode_qkv``), bitwise
equal to rope_kv_write followed by ``__call__``.
"""
import math

import torch

from . import _lib
from .linear import FragRows


def default_splits(batch, kv_heads, maximum, target_workgroups=512, min_keys=256, max_splits=16):
    """Split the key range only as far as needed to give the GPU about
    ``target_workgroups`` (batch * kv_heads * splits) workgroups, keeping at
    least ``min_keys`` keys per split; one split needs no combine pass."""
    want = math.ceil(target_workgroups / max(1, batch * kv_heads))
    return max(1, min(max_splits, want, maximum // min_keys))


class FlashDecode:
    def __init__(self, batch, kv_heads, groups, capacity, device, maximum=None, num_splits=None, ordered=False):
        if maximum is not None and not 0 < maximum <= capacity:
            raise ValueError("Decode attention requires a valid length bound")
        self.batch, self.kv_heads, self.groups, self.capacity = batch, kv_heads, groups, capacity
        self.maximum = capacity if maximum is None else maximum
        self.splits = num_splits or default_splits(batch, kv_heads, self.maximum)
        self.device = torch.device(device)
        size = _lib.size_query("lm_flash_decode_workspace_size", batch, kv_heads * groups, 64,
                               self.splits) if self.device.type == "cuda" else 0
        self.workspace = torch.empty(max(size, 1), dtype=torch.uint8, device=self.device)
        # ordered: a dispatch order (rows by descending length) the decode
        # prologue fills each step, for ragged batches (see fused_qkv).
        self.row_order = (torch.empty(batch, dtype=torch.int32, device=self.device)
                          if ordered and self.device.type == "cuda" else None)

    def __call__(self, q, k, v, lengths, active, scale, used=None):
        b, hq, s, d = q.shape
        if s != 1 or d != 64:
            raise ValueError("Decode attention takes one query position with head_dim 64")
        if k.shape != v.shape or k.shape[0] != b or k.shape[3] != d or hq % k.shape[1]:
            raise ValueError("KV cache layer shape does not match the queries")
        if b > self.batch or k.shape[2] != self.capacity:
            raise ValueError("Decode attention built for another batch/capacity")
        _lib.require_cuda(q, k, v, what="decode attention tensors")
        if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
            raise ValueError("Decode attention supports BF16")
        if q.stride(3) != 1 or not k.is_contiguous() or not v.is_contiguous():
            raise ValueError("Decode attention needs contiguous channels and cache layers")
        if used is None:
            used = torch.where(active, lengths + 1, 1).to(torch.int32)
        used = used.to(torch.int32).contiguous()
        out = torch.empty(b, hq, 1, d, device=q.device, dtype=q.dtype)
        _lib.call("lm_flash_decode", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(),
                  used.data_ptr(), b, hq, k.shape[1], self.capacity, d, float(scale), self.maximum,
                  self.splits, out.data_ptr(), self.workspace.data_ptr(), self.workspace.numel(),
                  _lib.stream(q.device))
        return out

    def fused_qkv(self, partials, cos_sin, positions, active, k, v, scale, used, q_heads, row_order=None,
                  frag_out=False):
        """Attention of one new token per row from the packed QKV projection's
        partials ``[S, B, (Hq + 2 Hkv) * 64]`` (litemoe/model.py:47-71 after
        the projection). Writes the rotated key and the value at
        ``positions[b]`` of ``k``/``v`` (rows with ``active`` false, when
        given, write nothing) and returns ``[B, Hq, 1, 64]``, or with
        ``frag_out`` the same values as a ``[B, Hq*64]``
        :class:`~litemoe_amd.linear.FragRows` (the o_proj split-K input
        order). ``row_order`` (int32 ``[B]``, a permutation of the rows) sets
        the order in which the rows' workgroups are dispatched; results do not
        depend on it."""
        splits, b, ncols = partials.shape
        hkv = k.shape[1]
        if ncols != (q_heads + 2 * hkv) * 64 or q_heads % hkv or k.shape != v.shape:
            raise ValueError("QKV partials do not match the cache heads")
        if b > self.batch or k.shape[0] < b or k.shape[2] != self.capacity or k.shape[3] != 64:
            raise ValueError("Decode attention built for another batch/capacity")
        _lib.require_cuda(partials, k, v, positions, used, what="decode attention tensors")
        if partials.dtype != torch.float32 or not partials.is_contiguous():
            raise ValueError("QKV partials must be contiguous fp32")
        if not k.is_contiguous() or not v.is_contiguous() or k.dtype != torch.bfloat16:
            raise ValueError("Decode attention needs contiguous BF16 cache layers")
        positions = positions.to(torch.int64).contiguous()
        used = used.to(torch.int32).contiguous()
        act = None
        if active is not None:
            # a bool mask is one byte per row: read it in place (no conversion launch)
            act = (active.view(torch.uint8) if active.dtype == torch.bool else active.to(torch.uint8)).contiguous()
        if frag_out:
            out = FragRows(b, q_heads * 64, k.device)
            out_ptr = out.data.data_ptr()
        else:
            out = torch.empty(b, q_heads, 1, 64, device=k.device, dtype=k.dtype)
            out_ptr = out.data_ptr()
        if row_order is not None and (row_order.dtype != torch.int32 or row_order.shape != (b,)):
            raise ValueError("row_order must be an int32 [B] permutation")
        _lib.call("lm_flash_decode_qkv_frag" if frag_out else "lm_flash_decode_qkv", partials.data_ptr(),
                  splits, cos_sin.data_ptr(), cos_sin.shape[0], positions.data_ptr(), _lib.ptr(act),
                  k.data_ptr(), v.data_ptr(), used.data_ptr(), _lib.ptr(row_order), b,
                  q_heads, hkv, self.capacity, 64, float(scale), self.maximum, self.splits,
                  out_ptr, self.workspace.data_ptr(), self.workspace.numel(), _lib.stream(k.device))
        return out
