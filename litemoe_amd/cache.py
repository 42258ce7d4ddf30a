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

    def write(self, layer, k, v, pos, active, slots=None):
        """Masked store of ``k, v [rows, H, 1, D]`` at ``(slots, h, pos)``
        (cache.py:50-55 -> kv_write.py:23-29)."""
        return kv_write.write(self, layer, k, v, pos, active, self.slots if slots is None else slots)


FusedKVCache = KVCache
