"""Granite MoE forward and greedy loop on the CPU — TEST INFRASTRUCTURE ONLY.

Restates litemoe/model.py:17-127 (forward, attention), cache.py:7-47 (KV
layout and decode masks), ep.py:42-53 (EP1 masking) and engine.py:87-148
(decode step, prefill state) for one process. Two rounding variants:

* ``fused=False`` — the reference CPU path: residual ``x + r * a``
  (model.py:108,122), bf16 router scales (model.py:117-118), expert combine
  by bf16 ``index_add_`` (ops.py:15-22), per-row decode GEMMs (ops.py:7-12).
* ``fused=True`` — the production (lean) rounding: ``x.add(a, alpha=r)``,
  fp32 scales, and the fp32 ordered combine of moe_finish.py:7-31.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import ops


class Cache:
    """litemoe/cache.py:7-19: ``k, v [L, B, Hkv, C, D]``."""

    def __init__(self, cfg, batch, capacity, dtype):
        self.capacity = capacity
        d = cfg.hidden_size // cfg.num_attention_heads
        shape = (cfg.num_hidden_layers, batch, cfg.num_key_value_heads, capacity, d)
        self.k = torch.zeros(shape, dtype=dtype)
        self.v = torch.zeros_like(self.k)


class Granite:
    def __init__(self, cfg, weights, capacity, fused=False):
        self.cfg, self.w, self.fused = cfg, weights, fused
        dtype = weights["embedding"].dtype
        d = cfg.hidden_size // cfg.num_attention_heads
        self.cos_sin, self.cos, self.sin = ops.rope_tables(cfg.rope_theta, d, capacity, dtype)

    # -- pieces ---------------------------------------------------------------
    def _residual(self, x, a):
        r = self.cfg.residual_multiplier
        return x.add(a, alpha=r) if self.fused else x + r * a

    def _qkv(self, z, w, single):
        cfg = self.cfg
        d = cfg.hidden_size // cfg.num_attention_heads
        t = z.shape[0]
        q = ops.linear_rows(z, w["self_attn.q_proj"], single).view(t, cfg.num_attention_heads, d)
        k = ops.linear_rows(z, w["self_attn.k_proj"], single).view(t, cfg.num_key_value_heads, d)
        v = ops.linear_rows(z, w["self_attn.v_proj"], single).view(t, cfg.num_key_value_heads, d)
        return q, k, v

    def _moe(self, z, w, valid, single):
        """Router (model.py:110-118) and experts (ep.py:42-53, ops.py:25-56)."""
        cfg = self.cfg
        scores = ops.linear_rows(z, w["block_sparse_moe.router.layer"], single)
        top, ids = ops.select_topk(scores, cfg.num_experts_per_tok)
        scales = top.softmax(-1)
        x = torch.where(valid[:, None], z, 0)
        if self.fused:
            return ops.fused_moe(x, ids.to(torch.int32), scales, w["input_linear"], w["output_linear"])
        scales = (scales.to(z.dtype).float() * valid[:, None])
        return ops.reference_experts(x, ids, scales, w["input_linear"], w["output_linear"], singleton=single)

    def _logits(self, x):
        cfg = self.cfg
        z = ops.rmsnorm(x, self.w["norm"], cfg.rms_norm_eps)
        return F.linear(z, self.w["head"]) / cfg.logits_scaling

    # -- prefill of one sequence into cache row ``slot`` -----------------------
    def prefill(self, prompt, cache, slot, last_only=False):
        """All-position logits ``[T, V]`` of one prompt (``[1, V]`` for the
        last position with ``last_only``); K/V of positions 0..T-1 go to cache
        row ``slot`` (cache.py:28-38 / packed.py)."""
        cfg = self.cfg
        tokens = torch.tensor(prompt)
        t = tokens.numel()
        pos = torch.arange(t)
        valid = torch.ones(t, dtype=torch.bool)
        x = F.embedding(tokens, self.w["embedding"]) * cfg.embedding_multiplier
        for layer, w in enumerate(self.w["layers"]):
            z = ops.rmsnorm(x, w["input_layernorm"], cfg.rms_norm_eps)
            q, k, v = self._qkv(z, w, False)
            q, k = ops.rope(q, self.cos, self.sin, pos), ops.rope(k, self.cos, self.sin, pos)
            cache.k[layer, slot, :, :t] = k.transpose(0, 1)
            cache.v[layer, slot, :, :t] = v.transpose(0, 1)
            cu = torch.tensor([0, t])
            a = ops.varlen_attention(q, k, v, cu, cfg.attention_multiplier).reshape(t, -1)
            x = self._residual(x, F.linear(a, w["self_attn.o_proj"]))
            z = ops.rmsnorm(x, w["post_attention_layernorm"], cfg.rms_norm_eps)
            x = self._residual(x, self._moe(z, w, valid, False))
        return self._logits(x[-1:] if last_only else x)

    # -- one decode step -------------------------------------------------------
    def decode(self, tokens, positions, valid, cache):
        """Logits ``[B, V]`` for one token per row (model.py:95-127 with
        slot=None): row b writes K/V at ``positions[b]`` if valid and attends
        keys ``0..positions[b]``; invalid rows attend key 0 and produce zeros
        from attention and experts (masked path)."""
        cfg = self.cfg
        b = tokens.numel()
        safe = torch.where(valid, positions, 0)
        x = F.embedding(tokens, self.w["embedding"]) * cfg.embedding_multiplier
        used = torch.where(valid, positions + 1, 1)
        for layer, w in enumerate(self.w["layers"]):
            z = ops.rmsnorm(x, w["input_layernorm"], cfg.rms_norm_eps)
            q, k, v = self._qkv(z, w, True)
            q, k = ops.rope(q, self.cos, self.sin, safe), ops.rope(k, self.cos, self.sin, safe)
            cache.k[layer], cache.v[layer] = ops.kv_store_rows(cache.k[layer], cache.v[layer], k, v, safe,
                                                               valid, torch.arange(b))
            a = ops.decode_attention(q, cache.k[layer], cache.v[layer], used, cfg.attention_multiplier)
            a = F.linear(a.reshape(b, -1), w["self_attn.o_proj"]) * valid[:, None]
            x = self._residual(x, a)
            z = ops.rmsnorm(x, w["post_attention_layernorm"], cfg.rms_norm_eps)
            x = self._residual(x, self._moe(z, w, valid, True))
        return self._logits(x)


def generate(model, prompts, budgets, capacity, ignore_eos=True, eos=None):
    """Greedy generation with the reference engine's state rules
    (engine.py:87-102 decode step, :128-148 / batch.py:53-64 prefill)."""
    batch = len(prompts)
    cache = Cache(model.cfg, batch, capacity, model.w["embedding"].dtype)
    outputs = [[] for _ in prompts]
    nxt = torch.zeros(batch, dtype=torch.int64)
    length = torch.tensor([len(p) for p in prompts])
    generated = torch.ones(batch, dtype=torch.int64)
    budget = torch.tensor(budgets)
    eos_ids = torch.tensor([] if eos is None else [eos])

    def is_eos(tok):
        return (tok[:, None] == eos_ids[None, :]).any(-1) if eos_ids.numel() else torch.zeros_like(tok, dtype=torch.bool)

    for j, p in enumerate(prompts):
        nxt[j] = model.prefill(p, cache, j)[-1].argmax(-1)
        outputs[j].append(int(nxt[j]))
    active = budget > 1
    if not ignore_eos:
        active &= ~is_eos(nxt)
    while bool(active.any()):
        valid = active.clone()
        positions = torch.where(valid, length, 0)
        candidate = model.decode(nxt, positions, valid, cache).argmax(-1)
        for j in range(batch):
            if valid[j]:
                outputs[j].append(int(candidate[j]))
        length += valid
        generated += valid
        nxt = torch.where(valid, candidate, nxt)
        done = generated >= budget
        if not ignore_eos:
            done |= is_eos(candidate)
        active = valid & ~done
    return outputs, cache
