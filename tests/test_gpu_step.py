"""The decode step's prologue and greedy epilogue kernels.

Bars: bit-exact against the reference's own torch ops for the same step
(litemoe/engine.py:87-102 around model.py:103-106 and :127) -- valid,
positions, ``used``, the scaled embedding and the first norm (the norm
against ``lm_rmsnorm``, which the oracle tests pin); the argmax (first index
of the maximum, NaN as maximum), the emit rows and every state tensor. At the
engine level, a lean step through the two kernels leaves the same emit rows,
state and KV cache as the reference-shaped step through ``forward``.
"""
import pytest
import torch
import torch.nn.functional as F

from litemoe_amd import _lib, norm, step
from litemoe_amd.synth import normal_bf16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def state_for(rows, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    length = torch.randint(0, 4000, (rows,), generator=g)
    generated = torch.randint(0, 6, (rows,), generator=g)
    budget = generated + torch.randint(0, 3, (rows,), generator=g)
    return {
        "next": torch.randint(0, vocab, (rows,), generator=g).to(DEV),
        "length": length.to(DEV),
        "generated": generated.to(DEV),
        "budget": budget.to(DEV),
        "active": (torch.rand(rows, generator=g) < 0.75).to(DEV),
        "present": torch.ones(rows, dtype=torch.bool, device=DEV),
    }


@pytest.mark.parametrize("rows,vocab,hidden", [(64, 49155, 1536), (3, 97, 256), (17, 1000, 1024),
                                               (5, 300, 4096), (2, 50, 8), (9, 64, 2048 + 8)])
@torch.inference_mode()
def test_prologue_equals_reference_ops(rows, vocab, hidden):
    s = state_for(rows, vocab, rows + hidden)
    table = normal_bf16((vocab, hidden), 0.5, hidden).to(DEV)
    weight = normal_bf16((hidden,), 0.3, 7).add(1).to(torch.bfloat16).to(DEV)
    mult, eps = 12.0, 1e-6
    x, z, valid, positions, used = step.decode_prologue(s["active"], s["length"], s["next"], table, mult,
                                                        weight, eps)
    ev = s["active"].clone()
    epos = torch.where(ev, s["length"], 0)
    assert torch.equal(valid, ev)
    assert torch.equal(positions, epos)
    assert torch.equal(used, (epos + 1).to(torch.int32))
    ex = F.embedding(s["next"], table) * mult
    assert torch.equal(x, ex)
    assert torch.equal(z, norm.rmsnorm(ex.contiguous(), weight, eps))


@pytest.mark.parametrize("rows", [1, 7, 64, 300])
@torch.inference_mode()
def test_prologue_row_order_is_stable_argsort_of_used(rows):
    """The dispatch order the prologue writes for the decode attention: rows
    by descending used, equal used by ascending row."""
    s = state_for(rows, 100, rows)
    s["length"] = (s["length"] % 7).to(DEV)  # many ties
    table = normal_bf16((100, 256), 0.5, 1).to(DEV)
    weight = torch.ones(256, dtype=torch.bfloat16, device=DEV)
    order = torch.full((rows,), -1, dtype=torch.int32, device=DEV)
    out = step.decode_prologue(s["active"], s["length"], s["next"], table, 1.0, weight, 1e-6, row_order=order)
    used = out[4].cpu().long()
    expect = torch.sort(-used, stable=True).indices.to(torch.int32)
    assert torch.equal(order.cpu(), expect)
    # and the other outputs are unchanged by it
    ref = step.decode_prologue(s["active"], s["length"], s["next"], table, 1.0, weight, 1e-6)
    for a, b in zip(out, ref):
        assert torch.equal(a, b)


@torch.inference_mode()
def test_prologue_limits():
    s = state_for(2, 10, 1)
    table = torch.zeros(10, 4104, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.NativeError):
        step.decode_prologue(s["active"], s["length"], s["next"], table, 1.0, table[0].clone(), 1e-6)
    table = torch.zeros(10, 20, dtype=torch.bfloat16, device=DEV)  # not a multiple of 8
    with pytest.raises(_lib.NativeError):
        step.decode_prologue(s["active"], s["length"], s["next"], table, 1.0, table[0].clone(), 1e-6)
    empty = {k: v[:0] for k, v in s.items()}
    out = step.decode_prologue(empty["active"], empty["length"], empty["next"], table[:, :16].contiguous(),
                               1.0, table[0, :16].clone(), 1e-6)
    assert out[0].shape == (0, 16)


def reference_step(logits, scaling, valid, s, emit, eos, ignore_eos):
    """litemoe/engine.py:92-102 on ``logits = raw / logits_scaling``."""
    candidate = (logits / scaling).argmax(-1)
    emit[:, 0].copy_(candidate)
    emit[:, 1].copy_(s["generated"])
    emit[:, 2].copy_(valid)
    s["length"].add_(valid)
    s["generated"].add_(valid)
    s["next"].copy_(torch.where(valid, candidate, s["next"]))
    done = s["generated"] >= s["budget"]
    if not ignore_eos and eos.numel():
        done = done | (candidate[:, None] == eos[None, :]).any(-1)
    s["active"].copy_(valid & ~done)


@pytest.mark.parametrize("rows,vocab", [(64, 49155), (3, 97), (33, 1000), (1, 1), (7, 5000)])
@pytest.mark.parametrize("scaling", [8.0, 3.7])
@pytest.mark.parametrize("ignore_eos", [False, True])
@torch.inference_mode()
def test_epilogue_equals_reference_step(rows, vocab, scaling, ignore_eos):
    seed = rows * 7 + vocab
    raw = normal_bf16((rows, vocab), 4.0, seed).to(DEV)
    g = torch.Generator().manual_seed(seed)
    # Planted ties: the row maximum at several indices (argmax takes the first).
    for r in range(0, rows, 2):
        idx = torch.randint(0, vocab, (3,), generator=g)
        raw[r, idx] = raw[r].max() + 1
    if rows > 2 and vocab > 4:
        raw[1, 3] = float("nan")  # NaN counts as the maximum
        raw[1, vocab - 1] = float("nan")
    s = state_for(rows, vocab, seed)
    eos_ids = [int(raw[0].argmax()) if vocab > 1 else 0, 11]
    for eos in (torch.tensor(eos_ids, dtype=torch.int64, device=DEV),
                torch.zeros(0, dtype=torch.int64, device=DEV)):
        exp_s = {k: v.clone() for k, v in s.items()}
        got_s = {k: v.clone() for k, v in s.items()}
        valid = s["active"].clone()
        exp_emit = torch.full((rows, 3), -5, dtype=torch.int64, device=DEV)
        got_emit = exp_emit.clone()
        reference_step(raw, scaling, valid, exp_s, exp_emit, eos, ignore_eos)
        step.greedy_epilogue(raw, scaling, valid, got_s, got_emit, eos, ignore_eos)
        assert torch.equal(got_emit, exp_emit)
        for k in s:
            assert torch.equal(got_s[k], exp_s[k]), k


@torch.inference_mode()
def test_epilogue_signed_zeros_infinities_and_negative_rows():
    """torch.argmax semantics on the edge values: -0 ties with +0 (first
    index wins), -inf rows, all-negative rows, NaN after a maximum, +inf."""
    vocab = 1003
    raw = torch.full((6, vocab), -3.0, dtype=torch.bfloat16)
    raw[0, 10], raw[0, 5] = 0.0, -0.0            # max 0: index 5 (-0) comes first
    raw[1, 7], raw[1, 900] = -0.0, 0.0           # max 0: index 7
    raw[2] = -float("inf")                       # all -inf: index 0
    raw[3] = -torch.arange(vocab, dtype=torch.float32).to(torch.bfloat16) - 1  # all negative: index 0
    raw[4, 400], raw[4, 401] = float("inf"), float("nan")  # NaN beats +inf
    raw[5, 999], raw[5, 2] = 5.0, 5.0            # tie: index 2
    raw = raw.to(DEV)
    s = state_for(6, vocab, 3)
    valid = torch.ones(6, dtype=torch.bool, device=DEV)
    eos = torch.zeros(0, dtype=torch.int64, device=DEV)
    exp_s = {k: v.clone() for k, v in s.items()}
    exp_emit = torch.zeros(6, 3, dtype=torch.int64, device=DEV)
    got_emit = exp_emit.clone()
    reference_step(raw, 6.0, valid, exp_s, exp_emit, eos, True)
    step.greedy_epilogue(raw, 6.0, valid, s, got_emit, eos, True)
    assert torch.equal(got_emit, exp_emit)
    assert got_emit[:, 0].tolist() == [5, 7, 0, 0, 401, 2]


@torch.inference_mode()
def test_epilogue_strided_logits():
    raw = normal_bf16((4, 3000), 2.0, 5).to(DEV)
    view = raw[:, :2999]  # row stride 3000
    s = state_for(4, 2999, 2)
    valid = s["active"].clone()
    eos = torch.zeros(0, dtype=torch.int64, device=DEV)
    exp_s = {k: v.clone() for k, v in s.items()}
    exp_emit = torch.zeros(4, 3, dtype=torch.int64, device=DEV)
    got_emit = exp_emit.clone()
    reference_step(view, 8.0, valid, exp_s, exp_emit, eos, False)
    step.greedy_epilogue(view, 8.0, valid, s, got_emit, eos, False)
    assert torch.equal(got_emit, exp_emit)
    for k in s:
        assert torch.equal(s[k], exp_s[k]), k


@pytest.mark.parametrize("hidden", [256, 1024])
@torch.inference_mode()
def test_lean_greedy_step_equals_forward_step(hidden):
    """One engine, two step paths: the kernels around the layers against the
    reference-shaped step (forward, then torch argmax and state update),
    compared after every step: emit rows, state and the KV cache."""
    from helpers import config_from_hf, hf_weights, make_hf
    from litemoe_amd.engine import Request
    from litemoe_amd.ep import ExpertParallel
    from litemoe_amd.experts import HipFusedExperts
    from litemoe_amd.model import Granite
    from litemoe_amd.optimized import OptimizedEngine, optimized_policy

    hf = make_hf(seed=4, vocab_size=301, hidden_size=hidden, intermediate_size=128, num_hidden_layers=2,
                 num_attention_heads=hidden // 64, num_key_value_heads=hidden // 128, num_local_experts=8,
                 num_experts_per_tok=2, max_position_embeddings=256, eos_token_id=5)
    cfg = config_from_hf(hf.config)
    w = hf_weights(hf, torch.bfloat16, DEV)
    ep = ExpertParallel(1, 0, 4096, cfg.hidden_size, cfg.num_experts_per_tok, torch.bfloat16, DEV,
                        HipFusedExperts())
    model = Granite(cfg, w, ep, 64)
    requests = [Request("a", [3, 8, 2], 9), Request("b", [4], 3), Request("c", [9, 2, 7, 7], 6),
                Request("d", [1], 1)]
    runs = [OptimizedEngine(model, requests, capacity=32) for _ in range(2)]
    for run in runs:
        run.prefill()
    assert torch.equal(runs[0].cache.k, runs[1].cache.k)
    supported = model.greedy_supported
    for _ in range(8):
        runs[0].decode_step()
        model.greedy_supported = lambda: False
        try:
            runs[1].decode_step()
        finally:
            model.greedy_supported = supported
        assert torch.equal(runs[0].emit, runs[1].emit)
        for k in runs[0].state:
            assert torch.equal(runs[0].state[k], runs[1].state[k]), k
        assert torch.equal(runs[0].cache.k, runs[1].cache.k)
        assert torch.equal(runs[0].cache.v, runs[1].cache.v)
    with optimized_policy(runs[0]):
        assert model.greedy_supported()
