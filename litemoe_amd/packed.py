"""Packed, ragged prefill: one row of all prompts with ``cu_seqlens``.

Mirrors litemoe/packed.py:6-36: ``PackedPrefill(cu, maximum, slots,
positions)`` with ``.attention(q, k, v, scale)`` (varlen causal attention,
here the gfx950 kernel) and ``packed_prefill_logits``.
"""
from typing import NamedTuple

import torch

from . import _lib


class PackedPrefill(NamedTuple):
    cu: torch.Tensor
    maximum: int
    slots: torch.Tensor
    positions: torch.Tensor

    def attention(self, q, k, v, scale):
        """``q [1, Hq, T, D]``, ``k, v [1, Hkv, T, D]`` (views) -> ``[T, Hq, D]``."""
        values = [x[0].transpose(0, 1) for x in (q, k, v)]
        return varlen_attention(*values, self.cu, self.maximum, scale, causal=True)


def varlen_attention(q, k, v, cu, maximum, scale, causal=True, out=None):
    """``q [T, Hq, 64]``, ``k, v [T, Hkv, 64]`` with contiguous channels."""
    _lib.require_cuda(q, k, v, cu, what="prefill attention tensors")
    if any(t.dtype != torch.bfloat16 or t.stride(-1) != 1 for t in (q, k, v)):
        raise ValueError('Prefill attention needs BF16 with contiguous channels')
    if q.shape[-1] != 64 or k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[1] % k.shape[1]:
        raise ValueError('Prefill attention shapes: q [T, Hq, 64], k/v [T, Hkv, 64]')
    cu = cu.to(torch.int32).contiguous()
    tokens, heads, dim = q.shape
    out = torch.empty(tokens, heads, dim, device=q.device, dtype=q.dtype) if out is None else out
    _lib.call("lm_prefill_attention", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0),
              k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), cu.data_ptr(), cu.numel() - 1, tokens,
              int(maximum), heads, k.shape[1], dim, float(scale), int(bool(causal)), out.data_ptr(),
              _lib.stream(q.device))
    return out


def build_packed(lengths, device, slot_start=0):
    """cu_seqlens, per-token positions and slots for prompts of ``lengths``
    (packed.py:25-33)."""
    if not lengths or min(lengths) < 1:
        raise ValueError("Packed Prefill requires nonempty prompts")
    ends = torch.tensor(lengths, dtype=torch.int32).cumsum(0, dtype=torch.int32)
    cu = torch.cat((ends.new_zeros(1), ends)).to(device)
    positions = torch.cat([torch.arange(n) for n in lengths]).to(device)
    slots = torch.cat([torch.full((n,), slot_start + i, dtype=torch.int64)
                       for i, n in enumerate(lengths)]).to(device)
    return PackedPrefill(cu, max(lengths), slots, positions), ends.to(device)


def packed_prefill_logits(model, prompts, cache, slot_start=0):
    """Prefill every prompt in one packed row; returns last-position logits
    ``[len(prompts), 1, V]`` (packed.py:19-36)."""
    if not cache.k.is_cuda:
        raise ValueError("Packed Prefill requires the GPU path")
    lengths = [len(p) for p in prompts]
    packed, ends = build_packed(lengths, cache.k.device, slot_start)
    tokens = torch.tensor([t for p in prompts for t in p], device=cache.k.device)[None]
    return model.forward(tokens, packed.positions[None], torch.ones_like(tokens, dtype=torch.bool),
                         cache, slot=packed, last=ends.long() - 1)
