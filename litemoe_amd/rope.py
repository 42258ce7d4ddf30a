"""Neox rotary embedding, alone or fused with the KV-cache store.

``rotary_embedding`` keeps the signature of vLLM's
``_custom_ops.rotary_embedding(positions, query, key, head_size, cos_sin_cache,
is_neox)`` as the reference calls it (litemoe/model.py:58,63-64): in place on
strided ``[T, heads, D]`` views. Arithmetic matches the torch path
``q * cos + rotate_half(q) * sin`` in bf16 (model.py:66-67) bit for bit.
"""
import torch

from . import _lib


def _check(q, k, cos_sin, positions):
    _lib.require_cuda(q, k, cos_sin, positions, what="RoPE tensors")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or cos_sin.dtype != torch.bfloat16:
        raise ValueError('RoPE supports BF16 query/key/table')
    if q.stride(-1) != 1 or k.stride(-1) != 1 or not cos_sin.is_contiguous():
        raise ValueError('RoPE needs contiguous channels and a contiguous cos/sin table')
    if q.shape[-1] != 64 or k.shape[-1] != 64 or cos_sin.shape[-1] != 64:
        raise ValueError('RoPE kernel supports head_dim 64')
    for t in (q, k):
        if t.stride(0) % 8 or t.stride(1) % 8 or t.data_ptr() % 16:
            raise ValueError('RoPE needs 16-byte aligned rows and heads (strides multiple of 8)')


def rotary_embedding(positions, query, key, head_size, cos_sin_cache, is_neox=True):
    """In-place neox rotation of ``query [T, Hq, D]`` and ``key [T, Hkv, D]``."""
    if not is_neox:
        raise ValueError('Only neox-style rotation is implemented (Granite)')
    if head_size != query.shape[-1]:
        raise ValueError('head_size must equal the last query dimension')
    _check(query, key, cos_sin_cache, positions)
    positions = positions.to(torch.int64).contiguous()
    rows = query.shape[0]
    _lib.call("lm_rope_kv_write", query.data_ptr(), query.stride(0), query.stride(1),
              key.data_ptr(), key.stride(0), key.stride(1), None, 0, 0,
              cos_sin_cache.data_ptr(), cos_sin_cache.shape[0], positions.data_ptr(), None, None,
              None, None, rows, query.shape[1], key.shape[1], 64, 1, 1, 1, _lib.stream(query.device))


def rope_kv_write(q, k, v, positions, active, cos_sin, cache, layer, slots=None, write_k=False):
    """Rotate ``q`` (in place) and ``k``, store rotated k and v into ``cache`` at
    ``(slots[r], h, positions[r])`` for active rows. ``q [T, Hq, 64]``,
    ``k, v [T, Hkv, 64]`` strided views (e.g. of the packed QKV projection).
    ``write_k`` also writes rotated k back in place (prefill attends over it).
    Replaces rotary_embedding + cache.write (litemoe/model.py:58-59, :64-70)."""
    _check(q, k, cos_sin, positions)
    kc, vc = cache.k[layer], cache.v[layer]
    if v.stride(-1) != 1 or v.dtype != torch.bfloat16 or kc.dtype != torch.bfloat16:
        raise ValueError('Fused RoPE/KV write needs BF16 v and cache with contiguous channels')
    if v.stride(0) % 8 or v.stride(1) % 8 or v.data_ptr() % 16:
        raise ValueError('RoPE needs 16-byte aligned v rows and heads (strides multiple of 8)')
    rows = q.shape[0]
    positions = positions.to(torch.int64).contiguous()
    active = active.to(torch.bool).contiguous()
    slots = None if slots is None else slots.to(torch.int64).contiguous()
    _lib.call("lm_rope_kv_write", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
              k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), cos_sin.data_ptr(),
              cos_sin.shape[0], positions.data_ptr(), active.data_ptr(), _lib.ptr(slots),
              kc.data_ptr(), vc.data_ptr(), rows, q.shape[1], k.shape[1], 64, cache.capacity,
              kc.shape[0], int(bool(write_k)), _lib.stream(q.device))
