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
    model.fused_head = False  # the head product as forward computes it (F.linear), for bitwise equality
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


@pytest.mark.parametrize("rows,vocab,hidden", [(64, 49155, 1536), (32, 49155, 1024), (128, 5003, 1536),
                                               (1, 97, 512), (17, 1000, 2048), (100, 777, 1024),
                                               (48, 16, 1536)])
@pytest.mark.parametrize("ignore_eos", [False, True])
@torch.inference_mode()
def test_head_greedy_equals_epilogue_on_its_logits(rows, vocab, hidden, ignore_eos):
    """lm_head_greedy against lm_greedy_epilogue (itself bit-exact against the
    reference's torch step) on the logits the fused head computes: the same
    candidates, emit rows and state bit for bit, with or without the logits
    stored. The logits against an fp32 product of the same bf16 operands:
    within one bf16 rounding (rtol 2^-7, atol 1e-3), rel-L2 <= 2e-2 as the
    north-star bar; the candidate is a maximum of the fp32 product's scaled
    values up to one bf16 ulp (the argmax of a different BLAS order may pick
    another index among near-ties, so agreement is reported, not required)."""
    seed = rows * 3 + vocab + hidden
    scaling = 8.0
    z = normal_bf16((rows, hidden), 1.0, seed).to(DEV)
    head = normal_bf16((vocab, hidden), 0.02, seed + 1)
    g = torch.Generator().manual_seed(seed)
    # planted ties: copies of one head row give equal logits at several indices
    for _ in range(4):
        src, dst = torch.randint(0, vocab, (2,), generator=g).tolist()
        head[dst] = head[src]
    head = head.to(DEV)
    s = state_for(rows, vocab, seed)
    valid = s["active"].clone()
    eos = torch.tensor([3, 11], dtype=torch.int64, device=DEV)
    logits = torch.full((rows, vocab), float("nan"), dtype=torch.bfloat16, device=DEV)
    got_s = {k: v.clone() for k, v in s.items()}
    exp_s = {k: v.clone() for k, v in s.items()}
    bare_s = {k: v.clone() for k, v in s.items()}
    got_emit = torch.full((rows, 3), -5, dtype=torch.int64, device=DEV)
    exp_emit, bare_emit = got_emit.clone(), got_emit.clone()
    packed = step.PackedHead(head)
    step.greedy_head(z, packed, scaling, valid, got_s, got_emit, eos, ignore_eos, logits_out=logits)
    step.greedy_epilogue(logits, scaling, valid, exp_s, exp_emit, eos, ignore_eos)
    step.greedy_head(z, packed, scaling, valid, bare_s, bare_emit, eos, ignore_eos)
    assert torch.equal(got_emit, exp_emit)
    assert torch.equal(bare_emit, exp_emit)
    for k in s:
        assert torch.equal(got_s[k], exp_s[k]), k
        assert torch.equal(bare_s[k], exp_s[k]), k
    ref = z.float() @ head.float().T
    got = logits.float()
    assert torch.allclose(got, ref, rtol=2 ** -7, atol=1e-3)
    assert float((got - ref).norm() / ref.norm()) <= 2e-2
    scaled = (ref.to(torch.bfloat16) / scaling).float()
    cand = got_emit[:, 0]
    picked = scaled.gather(1, cand[:, None])[:, 0]
    top = scaled.max(-1).values
    assert bool((picked >= top - top.abs() * 2 ** -6 - 1e-6).all())  # two bf16 roundings apart
    agree = int((cand == scaled.argmax(-1)).sum())
    print(f"head argmax agreement with the fp32 product: {agree}/{rows}")


@torch.inference_mode()
def test_head_greedy_ring_and_limits():
    """The emit ring slot written by the fused head path equals the emit
    rows; shapes without a kernel raise."""
    rows, vocab, hidden = 8, 300, 512
    z = normal_bf16((rows, hidden), 1.0, 1).to(DEV)
    head = normal_bf16((vocab, hidden), 0.02, 2).to(DEV)
    s = state_for(rows, vocab, 5)
    valid = s["active"].clone()
    eos = torch.zeros(0, dtype=torch.int64, device=DEV)
    emit = torch.zeros(rows, 3, dtype=torch.int64, device=DEV)
    host = torch.full((2, rows, 3), -1, dtype=torch.int64, pin_memory=True)
    import ctypes
    address = ctypes.c_void_p()
    _lib.call("lm_host_device_pointer", host.data_ptr(), ctypes.byref(address))
    counter = torch.full((1,), 2, dtype=torch.int64, device=DEV)  # step 2 -> slot 1
    step.greedy_head(z, step.PackedHead(head), 4.0, valid, s, emit, eos, True,
                     ring_target=(address.value, 2, counter))
    torch.cuda.synchronize()
    assert torch.equal(host[1], emit.cpu())
    assert bool((host[0] == -1).all())
    with pytest.raises(ValueError):
        step.greedy_head(z[:, :256].contiguous(), step.PackedHead(head[:, :256].contiguous()), 4.0, valid, s,
                         emit, eos, True)
    with pytest.raises(_lib.NativeError):
        nbytes = ctypes.c_int64()
        _lib.call("lm_head_greedy_workspace_size", 129, vocab, hidden, ctypes.byref(nbytes))


@torch.inference_mode()
def test_head_pack_layout():
    """lm_head_pack's chunk (k, tile, lane) is head[16*tile + lane%16][32*k + 8*(lane/16) .. +8], zero past
    the vocabulary."""
    vocab, hidden = 37, 512
    head = normal_bf16((vocab, hidden), 1.0, 3).to(DEV)
    packed = step.PackedHead(head).packed.view(hidden // 32, 3, 64, 8).cpu()
    h = torch.cat([head.cpu(), torch.zeros(48 - vocab, hidden, dtype=torch.bfloat16)])
    expect = h.view(3, 16, hidden // 32, 4, 8).permute(2, 0, 3, 1, 4).reshape(hidden // 32, 3, 64, 8)
    assert torch.equal(packed, expect)
