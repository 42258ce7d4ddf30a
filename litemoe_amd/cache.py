"""Contiguous rank-local KV cache ``[L, B, Hkv, C, D]`` (litemoe/cache.py:7-55).

The layout is the reference's: row b of the batch owns cache page b, a whole
``capacity``-long sequence per KV head. Writes go through the masked gfx950
store (one writer per row, head and channel)."""
import torch

from . import kv_write


class KVCache:
    def __init__(self, cfg, batch, capacity, device, dtype):
        self.capacity = capacity
        h, d = cfg.num_key_value_heads, cfg.hidden_size // cfg.num_attention_heads
        shape = (cfg.num_hidden_layers, batch, h, capacity, d)
        self.k = torch.zeros(shape, dtype=dtype, device=device)
        self.v = torch.zeros_like(self.k)
        self.keys = torch.arange(capacity, device=device)
        self.slots = torch.arange(batch, device=device)

    def reset(self):
        self.k.zero_()
        self.v.zero_()

    def prefill(self, layer, slot, k, v, valid):
        """Store a prefill's ``k, v`` and return ``(k, v, mask)``
        (litemoe/cache.py:21-33). ``slot`` a :class:`PackedPrefill`: ``k, v
        [1, H, T, D]`` go to ``(slot.slots[t], h, slot.positions[t])`` and the
        mask is None. ``slot`` an int or a slice: ``k, v [b, H, s, D]`` times
        ``valid [b, s]`` go to positions ``0 .. s-1`` of rows ``slot``; the
        mask ``[b, 1, s, s]`` is causal over valid keys, and a padding query
        sees key 0 only."""
        from .packed import PackedPrefill
        if isinstance(slot, PackedPrefill):
            tokens = k.shape[2]
            kv_write.write(self, layer, k[0].transpose(0, 1).unsqueeze(2), v[0].transpose(0, 1).unsqueeze(2),
                           slot.positions,
                           torch.ones(tokens, dtype=torch.bool, device=k.device), slot.slots)
            return k, v, None
        s = k.shape[2]
        rows = slot if isinstance(slot, slice) else slice(slot, slot + 1)
        keep = valid[:, None, :, None]
        self.k[layer, rows, :, :s].copy_(torch.where(keep, k, torch.zeros((), dtype=k.dtype, device=k.device)))
        self.v[layer, rows, :, :s].copy_(torch.where(keep, v, torch.zeros((), dtype=v.dtype, device=v.device)))
        pos = torch.arange(s, device=k.device)
        mask = (pos[:, None] >= pos[None, :])[None, None] & valid[:, None, None, :]
        mask = torch.where(valid[:, None, :, None], mask, (pos == 0)[None, None, None, :])
        return k, v, mask

    def decode(self, layer, k, v, lengths, active):
        """Masked store of one decode step's ``k, v [B, H, 1, D]`` at
        ``where(active, lengths, 0)``; returns the layer's cache and the key
        mask ``[B, 1, 1, C]`` (keys below ``lengths + 1``, key 0 for inactive
        rows), litemoe/cache.py:42-47."""
        pos = torch.where(active, lengths, 0)
        self.write(layer, k, v, pos, active)
        mask = self.keys[None, :] < (lengths + 1)[:, None]
        mask = torch.where(active[:, None], mask, self.keys[None, :] == 0)
        return self.k[layer], self.v[layer], mask[:, None, None, :]

    def write(self, layer, k, v, pos, active, slots=None):
        """Masked store of ``k, v [rows, H, 1, D]`` at ``(slots, h, pos)``
        (cache.py:50-55 -> kv_write.py:23-29)."""
        return kv_write.write(self, layer, k, v, pos, active, self.slots if slots is None else slots)


FusedKVCache = KVCache
