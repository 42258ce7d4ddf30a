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


def build_packed(lengths, device, slot_start=0, slots=None):
    """cu_seqlens, per-token positions and slots for prompts of ``lengths``
    (packed.py:25-33); sequence i goes to cache row ``slot_start + i``, or to
    ``slots[i]`` when a list of rows is given."""
    if not lengths or min(lengths) < 1:
        raise ValueError("Packed Prefill requires nonempty prompts")
    rows = [slot_start + i for i in range(len(lengths))] if slots is None else list(slots)
    if len(rows) != len(lengths):
        raise ValueError("Packed Prefill needs one cache row per prompt")
    ends = torch.tensor(lengths, dtype=torch.int32).cumsum(0, dtype=torch.int32)
    cu = torch.cat((ends.new_zeros(1), ends)).to(device)
    positions = torch.cat([torch.arange(n) for n in lengths]).to(device)
    slot_ids = torch.cat([torch.full((n,), row, dtype=torch.int64) for row, n in zip(rows, lengths)]).to(device)
    return PackedPrefill(cu, max(lengths), slot_ids, positions), ends.to(device)


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


def optimized_prefill_logits(model, prompts, cache, slot_start=0, max_tokens=1 << 17):
    """The prefill choice of litemoe/packed.py:39-51: packed when the model
    runs the lean prefill (or, for a batch, when the longest prompt is
    >= 1024 tokens or padding would add half again at >= 512), else one
    right-padded batch (:func:`litemoe_amd.batch.prefill_logits`). A packed
    prefill runs in chunks of at most ``max_tokens`` tokens (the expert
    workspace grows with the token count). Returns ``[len(prompts), 1, V]``."""
    from .batch import prefill_logits, prepare_batch
    if not cache.k.is_cuda:
        raise ValueError("Prefill runs on the GPU path only")
    lengths = [len(p) for p in prompts]
    width, batch = max(lengths), len(lengths)
    lean = getattr(model, "prefill_lean", False) and min(lengths) > 0
    if lean or (batch > 1 and min(lengths) > 0 and
                (width >= 1024 or (width >= 512 and 3 * sum(lengths) <= 2 * batch * width))):
        chunks, start = [], 0
        while start < batch:
            end, tokens = start + 1, lengths[start]
            while end < batch and tokens + lengths[end] <= max_tokens:
                tokens += lengths[end]
                end += 1
            prepare_batch(model, tokens)
            chunks.append(packed_prefill_logits(model, prompts[start:end], cache, slot_start + start))
            start = end
        return chunks[0] if len(chunks) == 1 else torch.cat(chunks)
    prepare_batch(model, batch * width)
    return prefill_logits(model, prompts, cache, slot_start)
