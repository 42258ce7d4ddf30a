"""Pins of the CPU oracle against independent references (no GPU).

Each oracle function is checked against something that does not share its
code: HF transformers' GraniteMoe implementation, torch's SDPA, brute force
over subsets, a counting sort, closed-form known answers, exact arithmetic on
bf16-exact inputs. A plausible mistake (a dropped term, a wrong sign, a
transposed operand, a wrong tie rule) fails one of them.
"""
import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import config_from_hf, hf_weights, make_hf, rel_l2
from oracle import granite, ops


# ------------------------------------------------------------ whole model --

@pytest.mark.parametrize("fused", [False, True])
@torch.inference_mode()
def test_oracle_prefill_and_incremental_logits_match_hf(tiny_hf, fused):
    """Reference test_core.py:86-99: fp32 logits equal HF within 2e-6/2e-5."""
    hf, cfg, w = tiny_hf
    model = granite.Granite(cfg, w, 16, fused=fused)
    cache = granite.Cache(cfg, 1, 16, torch.float32)
    tokens = [2, 5, 7, 9]
    logits = model.prefill(tokens, cache, 0)
    reference = hf(torch.tensor([tokens])).logits[0]
    torch.testing.assert_close(logits, reference, atol=2e-6, rtol=2e-5)
    token = int(reference[-1].argmax())
    actual = model.decode(torch.tensor([token]), torch.tensor([4]), torch.tensor([True]), cache)
    expected = hf(torch.tensor([tokens + [token]])).logits[:, -1]
    torch.testing.assert_close(actual, expected, atol=2e-6, rtol=2e-5)


@torch.inference_mode()
def test_oracle_greedy_matches_hf_with_ragged_batch(tiny_hf):
    """Reference test_core.py:102-121: greedy outputs equal HF greedy; rows
    stop at their budgets while others continue (masked decode rows)."""
    hf, cfg, w = tiny_hf
    prompts, budgets = [[3, 4, 8], [2], [9, 2, 6, 1, 5]], [4, 1, 3]
    outputs, _ = granite.generate(granite.Granite(cfg, w, 16), prompts, budgets, 16)
    for prompt, budget, got in zip(prompts, budgets, outputs):
        seq, expected = list(prompt), []
        for _ in range(budget):
            token = int(hf(torch.tensor([seq])).logits[0, -1].argmax())
            expected.append(token)
            seq.append(token)
        assert got == expected


@torch.inference_mode()
def test_oracle_bf16_decode_close_to_hf_bf16():
    """bf16 oracle vs HF bf16 (eager attention) on a 64-dim-head geometry,
    reference test_cuda_execution.py:136-165 tolerance (atol .002 rtol .02)
    scaled to these larger logits through rel-L2."""
    hf = make_hf(seed=3, vocab_size=97, hidden_size=256, intermediate_size=128, num_attention_heads=4,
                 num_key_value_heads=2, num_local_experts=8, num_experts_per_tok=2)
    cfg = config_from_hf(hf.config)
    model = granite.Granite(cfg, hf_weights(hf, torch.bfloat16), 32)
    hf = hf.to(torch.bfloat16)
    cache = granite.Cache(cfg, 1, 32, torch.bfloat16)
    tokens = [5, 17, 3, 44, 8, 90]
    got = model.prefill(tokens, cache, 0)
    ref = hf(torch.tensor([tokens])).logits[0]
    assert rel_l2(got, ref) < 2e-2


# ------------------------------------------------------------------ router --

def _brute_topk(row, k):
    """All k-subsets, ranked by (sum of values desc) then lexicographic ids,
    to find the top-k set; order within it by (value desc, id asc)."""
    values = [float(v) for v in row]
    best = max(itertools.combinations(range(len(values)), k),
               key=lambda c: (sorted((values[i] for i in c), reverse=True), [-i for i in sorted(c)]))
    return sorted(best, key=lambda i: (-values[i], i))


def test_select_topk_matches_brute_force_with_ties():
    rng = np.random.RandomState(0)
    for _ in range(200):
        e, k = rng.randint(2, 9), 0
        k = rng.randint(1, e + 1)
        row = torch.tensor(rng.randint(-3, 4, size=e), dtype=torch.float32).to(torch.bfloat16)
        _, ids = ops.select_topk(row[None], k)
        assert ids[0].tolist() == _brute_topk(row, k)


def test_route_weights_closed_form():
    rng = np.random.RandomState(1)
    logits = torch.tensor(rng.randn(16, 10), dtype=torch.float32).to(torch.bfloat16)
    for renorm in (True, False):
        weights, ids = ops.route(logits, 4, renormalize=renorm)
        for t in range(16):
            v = [float(x) for x in logits[t]]
            chosen = [v[i] for i in ids[t].tolist()]
            denom = sum(math.exp(c - max(v)) for c in (chosen if renorm else v))
            expected = [math.exp(c - max(v)) / denom for c in chosen]
            np.testing.assert_allclose(weights[t].numpy(), expected, rtol=2e-6)


def test_route_matches_hf_router():
    from transformers.models.granitemoe.modeling_granitemoe import GraniteMoeTopKRouter
    hf = make_hf()
    router = GraniteMoeTopKRouter(hf.config)
    torch.nn.init.normal_(router.weight)
    x = torch.randn(32, hf.config.hidden_size)
    ids, weights, logits = router(x)
    ours_w, ours_ids = ops.route(F.linear(x, router.weight), hf.config.num_experts_per_tok)
    assert torch.equal(ours_ids.long(), ids)
    torch.testing.assert_close(ours_w, weights.float(), rtol=1e-6, atol=1e-7)


def test_permutation_matches_counting_sort():
    rng = np.random.RandomState(2)
    for _ in range(50):
        local, first = rng.randint(1, 12), rng.randint(0, 4)
        ids = torch.tensor(rng.randint(0, local + first + 3, size=(rng.randint(1, 40), 3)))
        offsets, order, inverse = ops.permutation(ids, local, first)
        buckets = [[] for _ in range(local + 1)]
        for r, e in enumerate(ids.flatten().tolist()):
            key = e - first
            buckets[key if 0 <= key < local else local].append(r)
        assert order.tolist() == [r for b in buckets for r in b]
        assert offsets.tolist() == list(itertools.accumulate([0] + [len(b) for b in buckets[:-1]]))
        assert all(order[inverse[r]] == r for r in range(order.numel()))


# ----------------------------------------------------------------- experts --

KNOWN = dict(x=[[1., 2.], [2., 1.]], ids=[[0, 1], [1, 0]], scales=[[.25, .75], [.1, .9]])
# out[t] = sum_j s[t,j] * W2[e] (silu(W13[e,:2] x_t) * W13[e,2:] x_t) with
# W13 = arange(16)/20 as [2,4,2], W2 = arange(8)/20 as [2,2,2], evaluated with
# scalar float64 arithmetic.
KNOWN_OUT = [[0.8432774337062205, 1.2154118081694232], [0.11345300938746344, 0.17797190472437896]]


def test_reference_experts_known_answer_and_invariants():
    """Reference test_core.py:22-36 example with its hand-computed answer."""
    x = torch.tensor(KNOWN["x"], dtype=torch.float64)
    w1 = torch.arange(16, dtype=torch.float64).view(2, 4, 2) / 20
    w2 = torch.arange(8, dtype=torch.float64).view(2, 2, 2) / 20
    ids = torch.tensor(KNOWN["ids"])
    scales = torch.tensor(KNOWN["scales"], dtype=torch.float64)
    out = ops.reference_experts(x, ids, scales, w1, w2)
    np.testing.assert_allclose(out.numpy(), KNOWN_OUT, rtol=1e-12)
    parts = sum(ops.reference_experts(x, ids, scales, w1[r:r + 1], w2[r:r + 1], r, 2) for r in range(2))
    torch.testing.assert_close(parts, out)
    torch.testing.assert_close(ops.reference_experts(x, ids, scales * 2, w1, w2), out * 2)
    nan = torch.full_like(x, float("nan"))
    ops.reference_experts(x, torch.ones_like(ids), scales, w1[:1], w2[:1], 0, 2, nan)
    assert torch.equal(nan, torch.zeros_like(nan))
    fused = ops.fused_moe(x, ids.int(), scales, w1, w2)  # fp32 combine accumulator
    np.testing.assert_allclose(fused.numpy(), KNOWN_OUT, rtol=1e-6)


def test_expert_routes_and_fused_match_hf_experts():
    """HF GraniteMoeExperts (its own per-expert loop) on fp32 random data."""
    hf = make_hf(seed=11, hidden_size=64, intermediate_size=32, num_local_experts=6, num_experts_per_tok=3)
    experts = hf.model.layers[0].block_sparse_moe.experts
    torch.nn.init.normal_(experts.gate_up_proj, std=0.2)
    torch.nn.init.normal_(experts.down_proj, std=0.2)
    x = torch.randn(20, 64)
    logits = torch.randn(20, 6)
    top, ids = logits.topk(3, -1)
    w = top.softmax(-1)
    with torch.no_grad():
        expected = experts(x, ids, w)
        got = ops.fused_moe(x, ids.int(), w, experts.gate_up_proj.data, experts.down_proj.data)
        ref = ops.reference_experts(x, ids, w, experts.gate_up_proj.data, experts.down_proj.data)
    torch.testing.assert_close(got, expected, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(ref, expected, atol=1e-5, rtol=1e-5)


def test_finish_exact_on_bf16_exact_inputs_and_order():
    """Integer y and power-of-two scales: every product and partial sum is
    exact, so the ordered fp32 sum equals the exact integer sum."""
    rng = np.random.RandomState(3)
    batch, k, hidden, experts = 7, 4, 33, 9
    ids = torch.stack([torch.randperm(experts)[:k] for _ in range(batch)]).int()
    y = torch.tensor(rng.randint(-64, 64, size=(batch * k, hidden)), dtype=torch.float32).to(torch.bfloat16)
    scales = torch.tensor(2.0 ** rng.randint(-3, 2, size=(batch, k)), dtype=torch.float32)
    out = ops.finish(y, ids, scales, 0, experts)
    exact = (y.double().view(batch, k, hidden) * scales.double()[..., None]).sum(1)
    assert torch.equal(out.double(), exact.to(torch.bfloat16).double())
    # y given in sorted order through the inverse permutation gives the same
    offsets, order, inverse = ops.permutation(ids, experts)
    assert torch.equal(ops.finish(y[order], ids, scales, 0, experts, inverse=inverse), out)


def test_finish_skips_non_owned_and_matches_combine():
    """Reference test_moe_finish.py semantics: non-owned rows never read
    (NaN-poisoned), zero-scale rows give exact zeros, rel-L2 <= 0.01 vs combine."""
    torch.manual_seed(29)
    for batch, topk, hidden, rank, world, remap in [(8, 8, 129, 0, 1, False), (8, 3, 65, 1, 2, True),
                                                    (32, 8, 65, 1, 2, False)]:
        count = 8
        ids = torch.stack([torch.randperm(count * world)[:topk] for _ in range(batch)]).int()
        order = ids.flatten().argsort()
        y = torch.randn(batch * topk, hidden).to(torch.bfloat16)
        scales = torch.softmax(torch.randn(batch, topk), -1)
        scales[-1] = 0
        logical = torch.randperm(count * world) if remap else None
        selected = ids.flatten()[order].long() - rank * count
        owned = (selected >= 0) & (selected < count)
        weighted = torch.where(owned[:, None], y, 0) * scales.flatten()[order, None].to(y.dtype)
        expected = ops.combine(torch.zeros(batch, hidden, dtype=torch.bfloat16), ids, order, weighted, logical)
        y[~owned] = float("nan")
        inverse = torch.empty_like(order)
        inverse[order] = torch.arange(order.numel())
        out = ops.finish(y, ids, scales, rank, count, logical, inverse=inverse)
        assert torch.isfinite(out).all()
        assert rel_l2(out, expected) <= 0.01
        assert torch.count_nonzero(out[-1]) == 0


# ------------------------------------------------- norm / rope / kv / attn --

def test_rmsnorm_matches_hf_bitwise():
    from transformers.models.granitemoe.modeling_granitemoe import GraniteMoeRMSNorm
    for dtype in (torch.float32, torch.bfloat16):
        norm = GraniteMoeRMSNorm(1536, eps=1e-6)
        with torch.no_grad():
            norm.weight.copy_(1 + 0.2 * torch.randn(1536))
        norm = norm.to(dtype)
        x = (torch.randn(8, 1536) * 3).to(dtype)
        with torch.no_grad():
            assert torch.equal(ops.rmsnorm(x, norm.weight.data, 1e-6), norm(x))


@pytest.mark.parametrize("theta", [10000.0, 1000000.0])
def test_rope_tables_and_rotation_match_hf(theta):
    """Reference test_cuda_execution.py:12-28 and test_native_rope_entry.py:
    28-48 (tables bitwise through position 4095), plus HF's rotation."""
    from transformers import GraniteMoeConfig
    from transformers.models.granitemoe.modeling_granitemoe import (GraniteMoeRotaryEmbedding,
                                                                    apply_rotary_pos_emb)
    cfg = GraniteMoeConfig(hidden_size=1024, num_attention_heads=16, num_key_value_heads=8,
                           rope_parameters=dict(rope_type="default", rope_theta=theta))
    cfg.rope_theta = theta
    dummy = torch.zeros(1, 1, dtype=torch.bfloat16)
    cos, sin = GraniteMoeRotaryEmbedding(cfg)(dummy, torch.arange(4096)[None])
    cos_sin, ocos, osin = ops.rope_tables(theta, 64, 4096, torch.bfloat16)
    assert torch.equal(ocos, cos[0]) and torch.equal(osin, sin[0])
    assert torch.equal(cos_sin, torch.cat((cos[0][:, :32], sin[0][:, :32]), -1))
    pos = torch.randint(0, 4096, (5,))
    q = torch.randn(5, 16, 64).to(torch.bfloat16)
    k = torch.randn(5, 8, 64).to(torch.bfloat16)
    hq, hk = apply_rotary_pos_emb(q.transpose(0, 1), k.transpose(0, 1), cos[0][pos], sin[0][pos], unsqueeze_dim=0)
    assert torch.equal(ops.rope(q, ocos, osin, pos), hq.transpose(0, 1))
    assert torch.equal(ops.rope(k, ocos, osin, pos), hk.transpose(0, 1))


def test_kv_store_matches_flat_index_formula():
    """The loop store vs the reference kernel's flat target index
    ((slot*H + h)*C + pos)*D + c (kv_write.py:16), incl. inactive and
    out-of-range rows (test_cache_write.py:7-33 cases)."""
    torch.manual_seed(5)
    batch, heads, cap, dim = 3, 2, 8, 4
    kc, vc = torch.randn(batch, heads, cap, dim), torch.randn(batch, heads, cap, dim)
    k, v = torch.randn(3, heads, dim), torch.randn(3, heads, dim)
    k[1] = float("nan")
    positions = torch.tensor([0, cap + 10, cap - 1])
    active = torch.tensor([True, False, True])
    slots = torch.tensor([2, 1, 0])
    nk, nv = ops.kv_store(kc, vc, k, v, positions, active, slots)
    rk, rv = ops.kv_store_rows(kc, vc, k, v, positions, active, slots)
    assert torch.equal(rk, nk) and torch.equal(rv, nv)
    ek, ev = kc.clone().view(-1), vc.clone().view(-1)
    for row in (0, 2):
        for h in range(heads):
            for c in range(dim):
                target = ((int(slots[row]) * heads + h) * cap + int(positions[row])) * dim + c
                ek[target], ev[target] = k[row, h, c], v[row, h, c]
    assert torch.equal(nk.view(-1), ek) and torch.equal(nv.view(-1), ev)


def test_decode_attention_matches_sdpa():
    torch.manual_seed(6)
    b, hq, hkv, cap, d = 4, 6, 2, 40, 64
    q = torch.randn(b, hq, d)
    kc, vc = torch.randn(b, hkv, cap, d), torch.randn(b, hkv, cap, d)
    used = torch.tensor([1, 17, 40, 5])
    got = ops.decode_attention(q, kc, vc, used, 0.125)
    mask = torch.arange(cap)[None, :] < used[:, None]
    ref = F.scaled_dot_product_attention(q[:, :, None], kc.repeat_interleave(3, 1), vc.repeat_interleave(3, 1),
                                         attn_mask=mask[:, None, None, :], scale=0.125)[:, :, 0]
    torch.testing.assert_close(got, ref, atol=1e-5, rtol=1e-5)


def test_varlen_attention_matches_sdpa_per_sequence():
    """Reference test_packed_prefill.py:28-44 in fp32 on the CPU."""
    torch.manual_seed(11)
    q = torch.randn(9, 4, 64)
    k, v = torch.randn(9, 2, 64), torch.randn(9, 2, 64)
    cu = torch.tensor([0, 2, 9])
    got = ops.varlen_attention(q, k, v, cu, 0.125)
    parts = []
    for l, r in [(0, 2), (2, 9)]:
        parts.append(F.scaled_dot_product_attention(
            q[l:r].transpose(0, 1), k[l:r].transpose(0, 1).repeat_interleave(2, 0),
            v[l:r].transpose(0, 1).repeat_interleave(2, 0), is_causal=True, scale=0.125).transpose(0, 1))
    torch.testing.assert_close(got, torch.cat(parts), atol=1e-5, rtol=1e-5)


def test_varlen_attention_non_causal_and_empty_sequence_match_sdpa():
    """The non-causal branch (every token of a sequence attends every key of
    it) against SDPA without a mask, per sequence, with an empty sequence
    inside the pack and three q heads per kv head."""
    torch.manual_seed(12)
    q = torch.randn(12, 6, 64)
    k, v = torch.randn(12, 2, 64), torch.randn(12, 2, 64)
    cu = torch.tensor([0, 5, 5, 12])
    got = ops.varlen_attention(q, k, v, cu, 0.125, causal=False)
    parts = []
    for l, r in [(0, 5), (5, 12)]:
        parts.append(F.scaled_dot_product_attention(
            q[l:r].transpose(0, 1), k[l:r].transpose(0, 1).repeat_interleave(3, 0),
            v[l:r].transpose(0, 1).repeat_interleave(3, 0), is_causal=False, scale=0.125).transpose(0, 1))
    torch.testing.assert_close(got, torch.cat(parts), atol=1e-5, rtol=1e-5)
    # the causal and non-causal results agree on each sequence's last token only
    causal = ops.varlen_attention(q, k, v, cu, 0.125)
    torch.testing.assert_close(causal[[4, 11]], got[[4, 11]], atol=1e-6, rtol=1e-6)
    assert not torch.allclose(causal[[0, 5]], got[[0, 5]])
