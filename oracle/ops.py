"""Operator semantics of the reference hot path, restated on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Every function cites the
reference lines it restates (paths relative to the reference repository).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def linear_rows(x, weight, singleton=False):
    """litemoe/ops.py:7-12: per-row F.linear when ``singleton`` (decode shape)."""
    if singleton and x.numel() // x.shape[-1] > 1:
        rows = x.reshape(-1, x.shape[-1]).split(1)
        return torch.cat([F.linear(row, weight) for row in rows]).view(*x.shape[:-1], weight.shape[0])
    return F.linear(x, weight)


def rmsnorm(x, weight, eps):
    """litemoe/model.py:9-11 (and norm.py:15): the bf16 cast before the weight."""
    z = x.float()
    return (z * torch.rsqrt(z.square().mean(-1, keepdim=True) + eps)).to(x.dtype) * weight


def rotate_half(x):
    """litemoe/model.py:13-15."""
    a, b = x.chunk(2, dim=-1)
    return torch.cat((-b, a), dim=-1)


def rope_tables(theta, dim, capacity, dtype, device="cpu"):
    """litemoe/model.py:31-36: (cos_sin, cos, sin) tables."""
    inv = 1.0 / theta ** (torch.arange(0, dim, 2, device="cpu").float() / dim)
    freq = torch.outer(torch.arange(capacity, device=device).float(), inv.to(device))
    cos_sin = torch.cat((freq.cos(), freq.sin()), -1).to(dtype)
    cos, sin = [half.repeat(1, 2) for half in cos_sin.chunk(2, -1)]
    return cos_sin, cos, sin


def rope(x, cos, sin, positions):
    """litemoe/model.py:66-67 on ``x [T, H, D]`` with positions ``[T]``."""
    c, s = cos[positions][:, None], sin[positions][:, None]
    return x * c + rotate_half(x) * s


# ------------------------------------------------------------------ routing --

def select_topk(logits, k):
    """Top-k ids in descending logit order, equal logits by ascending id.

    The reference CPU path calls ``scores.float().topk(k)`` (litemoe/model.py:115)
    whose tie order is implementation-defined; this fixes the stable rule.
    Returns (values fp32, ids int64)."""
    values = logits.float()
    order = torch.sort(-values, dim=-1, stable=True).indices[..., :k]
    return values.gather(-1, order), order


def route(logits, k, renormalize=True):
    """Router outputs from bf16 logits: fp32 weights and int32 ids.

    renormalize: softmax over the k selected (litemoe/model.py:115-116; HF
    modeling_granitemoe.py GraniteMoeTopKRouter.forward); otherwise the softmax
    over all logits taken at the selection (vLLM fused_topk renormalize=False)."""
    top, ids = select_topk(logits, k)
    if renormalize:
        weights = top.softmax(-1)
    else:
        weights = logits.float().softmax(-1).gather(-1, ids)
    return weights, ids.to(torch.int32)


def permutation(ids, local, first=0):
    """Stable expert-sorted permutation of flat routes (litemoe/ops.py:163-173
    with a stable sort): returns offsets [local+1], sorted routes, inverse."""
    flat = ids.reshape(-1).long() - first
    key = torch.where((flat >= 0) & (flat < local), flat, local)
    order = torch.sort(key, stable=True).indices
    counts = torch.bincount(key, minlength=local + 1)
    offsets = torch.zeros(local + 1, dtype=torch.int64)
    offsets[1:] = counts[:local].cumsum(0)
    inverse = torch.empty_like(order)
    inverse[order] = torch.arange(order.numel())
    return offsets, order, inverse


# ------------------------------------------------------------------ experts --

def combine(out, ids, order, weighted, logical=None):
    """litemoe/ops.py:15-22: one bf16 index_add in expert-sorted order."""
    if logical is not None:
        routes = weighted.new_zeros((ids.numel(), weighted.shape[-1]))
        routes.index_copy_(0, order, weighted)
        order = logical[ids].to(ids.dtype).flatten().argsort()
        weighted = routes[order]
    return out.index_add_(0, order // ids.shape[1], weighted)


def reference_experts(x, ids, scales, w1, w2, rank=0, world=1, out=None, logical=None, routes=False,
                      singleton=False, stable=True):
    """litemoe/ops.py:25-56. ``stable`` uses argsort(stable=True) for the
    route order; the reference's unstable argsort only permutes routes of the
    same expert, which changes no GEMM row and (in fp32) no sum."""
    if out is None:
        out = x.new_zeros((*ids.shape, x.shape[-1])) if routes else torch.zeros_like(x)
    else:
        out.zero_()
    start = rank * w1.shape[0]
    order = ids.flatten().argsort(stable=stable)
    token, branch = order // ids.shape[1], order % ids.shape[1]
    counts = torch.zeros(w1.shape[0] * world, dtype=torch.int32)
    counts.scatter_add_(0, ids.flatten().long(), torch.ones_like(order, dtype=torch.int32))
    sizes = counts.tolist()
    grouped = x[token].split(sizes)
    all_outputs = []
    for local, rows in enumerate(grouped[start:start + w1.shape[0]]):
        if rows.shape[0]:
            gate, up = linear_rows(rows, w1[local], singleton).chunk(2, -1)
            all_outputs.append(linear_rows(F.silu(gate) * up, w2[local], singleton))
    if all_outputs:
        begin, length = sum(sizes[:start]), sum(sizes[start:start + w1.shape[0]])
        selected, selected_branch = token[begin:begin + length], branch[begin:begin + length]
        weighted = torch.cat(all_outputs) * scales[selected, selected_branch, None].to(x.dtype)
        if routes:
            out.view(-1, x.shape[1]).index_copy_(0, order[begin:begin + length], weighted)
        else:
            combine(out, ids, order[begin:begin + length], weighted, logical)
    return out


def expert_routes(x, ids, w1, w2):
    """Per-route expert outputs in route order ``r = t*K + j`` (bf16 [M*K, H]):
    the per-row expert math of litemoe/ops.py:43-47 (gate/up, silu, product and
    W2 output each rounded to the input dtype)."""
    k = ids.shape[1]
    flat = ids.reshape(-1).long()
    y = torch.empty(flat.numel(), w2.shape[1], dtype=x.dtype)
    for e in flat.unique().tolist():
        routes = (flat == e).nonzero().flatten()
        rows = x[routes // k]
        gate, up = F.linear(rows, w1[e]).chunk(2, -1)
        y[routes] = F.linear(F.silu(gate) * up, w2[e])
    return y


def finish(y, ids, scales, rank=0, count=None, logical=None, inverse=None):
    """litemoe/moe_finish.py:7-31: per token, routes in ascending
    (logical id * K + branch) order, ``total += bf16(bf16(y) * bf16(scale))``
    in fp32; non-owned routes are never read. ``y`` rows are in route order,
    or in sorted order when ``inverse`` (route -> row) is given."""
    batch, k = ids.shape
    count = ids.max().item() + 1 if count is None else count
    out = torch.zeros(batch, y.shape[1], dtype=torch.float32)
    for t in range(batch):
        e = ids[t].long()
        key = (logical[e] if logical is not None else e) * k + torch.arange(k)
        for j in torch.argsort(key).tolist():
            r = t * k + j
            if not 0 <= e[j].item() - rank * count < count:
                continue
            row = inverse[r].item() if inverse is not None else r
            s = scales[t, j].to(y.dtype).float()
            out[t] += (y[row].float() * s).to(y.dtype).float()
    return out.to(y.dtype)


def fused_moe(x, ids, scales, w1, w2, logical=None):
    """The fused experts of the decode path: ``finish(expert_routes(...))``."""
    return finish(expert_routes(x, ids, w1, w2), ids, scales, 0, w1.shape[0], logical)


# ---------------------------------------------------------------- KV cache --

def kv_store(kc, vc, k, v, positions, active, slots):
    """litemoe/kv_write.py:12-20 element by element: for active rows,
    ``KC[slot, h, pos, c] = K[row, h, c]`` (target index kv_write.py:16)."""
    kc, vc = kc.clone(), vc.clone()
    batch, heads, capacity, dim = kc.shape
    for row in range(k.shape[0]):
        if not bool(active[row]):
            continue
        p, slot = int(positions[row]), int(slots[row])
        if not (0 <= p < capacity and 0 <= slot < batch):
            continue
        for h in range(heads):
            for c in range(dim):
                kc[slot, h, p, c] = k[row, h, c]
                vc[slot, h, p, c] = v[row, h, c]
    return kc, vc


def kv_store_rows(kc, vc, k, v, positions, active, slots):
    """Row-wise form of :func:`kv_store` (one slice assignment per stored row);
    same semantics, fast enough for benchmark-sized caches."""
    kc, vc = kc.clone(), vc.clone()
    batch, _, capacity, _ = kc.shape
    for row in range(k.shape[0]):
        p, slot = int(positions[row]), int(slots[row])
        if bool(active[row]) and 0 <= p < capacity and 0 <= slot < batch:
            kc[slot, :, p] = k[row]
            vc[slot, :, p] = v[row]
    return kc, vc


# --------------------------------------------------------------- attention --

def decode_attention(q, kc, vc, used, scale):
    """Row b attends keys ``j < used[b]`` of its cache page (litemoe/
    flash_decode.py:16-22, masks cache.py:42-47). ``q [B, Hq, D]``,
    ``kc, vc [B, Hkv, C, D]``; fp32 math, output in q's dtype."""
    b, hq, d = q.shape
    g = hq // kc.shape[1]
    out = torch.zeros(b, hq, d, dtype=torch.float32)
    for row in range(b):
        n = int(used[row])
        if n <= 0:
            continue
        keys = kc[row, :, :n].float().repeat_interleave(g, 0)
        values = vc[row, :, :n].float().repeat_interleave(g, 0)
        s = torch.einsum("hd,hjd->hj", q[row].float(), keys) * scale
        out[row] = torch.einsum("hj,hjd->hd", s.softmax(-1), values)
    return out.to(q.dtype)


def varlen_attention(q, k, v, cu, scale, causal=True):
    """Packed attention (litemoe/packed.py:12-16): sequence s owns tokens
    [cu[s], cu[s+1]); token i attends keys 0..i (causal). ``q [T, Hq, D]``,
    ``k, v [T, Hkv, D]``; fp32 math."""
    out = torch.zeros(q.shape, dtype=torch.float32)
    g = q.shape[1] // k.shape[1]
    for s in range(cu.numel() - 1):
        a, b = int(cu[s]), int(cu[s + 1])
        if b <= a:
            continue
        qq = q[a:b].float().transpose(0, 1)
        kk = k[a:b].float().transpose(0, 1).repeat_interleave(g, 0)
        vv = v[a:b].float().transpose(0, 1).repeat_interleave(g, 0)
        s_ = qq @ kk.transpose(1, 2) * scale
        if causal:
            n = b - a
            s_ = s_.masked_fill(torch.ones(n, n, dtype=torch.bool).triu(1), float("-inf"))
        out[a:b] = (s_.softmax(-1) @ vv).transpose(0, 1)
    return out.to(q.dtype)
