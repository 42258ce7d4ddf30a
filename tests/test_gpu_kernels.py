"""Kernel-level parity of the gfx950 path against the CPU oracle.

Bars: bit-exact for integer/index work (top-k ids given logits, the route
permutation, KV stores, RoPE, the combine given y); floating point within the
tolerances written in each test (the reference's own where it has one,
otherwise the rel-L2 <= 2e-2 of the north star).
"""
import pytest
import torch

from helpers import rel_l2
from litemoe_amd import experts, flash_decode, kv_write, moe_finish, norm, packed, rope, router
from litemoe_amd.cache import KVCache
from litemoe_amd.config import ModelConfig
from litemoe_amd.synth import normal_bf16
from oracle import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf(shape, std=1.0, seed=0):
    return normal_bf16(shape, std, seed)


def ordered(t):
    """bf16 bit patterns on a monotone integer line (-0 and +0 coincide)."""
    i = t.contiguous().view(torch.int16).to(torch.int32)
    return torch.where(i >= 0, i, -(i & 0x7FFF))


def ulp_diff(a, b):
    """Max distance between bf16 tensors in units in the last place."""
    return int((ordered(a) - ordered(b)).abs().max()) if a.numel() else 0


def within_ulp_or_abs(a, b, ulps, floor):
    """Every element within ``ulps`` bf16 ulps, or within ``floor`` absolutely
    (dot products near zero lose relative accuracy to cancellation)."""
    close = (ordered(a) - ordered(b)).abs() <= ulps
    return bool((close | ((a.float() - b.float()).abs() <= floor)).all())


# ------------------------------------------------------------------- norms --

@pytest.mark.parametrize("shape", [(1, 1, 1536), (8, 1, 2048), (32, 1, 3072), (2, 1, 33), (64, 1, 1536)])
@torch.inference_mode()
def test_rmsnorm_matches_oracle(shape):
    x = bf(shape, 1.0, 1)
    w = (1 + 0.2 * bf(shape[-1:], 1.0, 2).float()).to(torch.bfloat16)
    for scale in (0.0, 1e-3, 1.0, 1e3):
        xs = (x.float() * scale).to(torch.bfloat16)
        got = norm.rmsnorm(xs.to(DEV), w.to(DEV), 1e-6).cpu()
        exp = ops.rmsnorm(xs, w, 1e-6)
        torch.testing.assert_close(got, exp, atol=.016, rtol=.008)  # reference test_fused_norm.py:97
        if scale:
            assert rel_l2(got, exp) < .005
            assert (got != exp).float().mean() < 0.01  # rsqrt rounding flips at most a few ulps


@torch.inference_mode()
def test_add_rmsnorm_updates_residual_and_normalises():
    x = bf((64, 1536), 1.0, 3)
    a = bf((64, 1536), 1.0, 4)
    w = (1 + 0.2 * bf((1536,), 1.0, 5).float()).to(torch.bfloat16)
    xd = x.to(DEV)
    y = norm.add_rmsnorm(xd, a.to(DEV), 0.22, w.to(DEV), 1e-6).cpu()
    # alpha stays fp32 (the CUDA add with alpha computes in fp32 opmath)
    x_new = (x.double() + 0.22 * a.double()).to(torch.bfloat16)
    # near-exact cancellation (x ~ -0.22 a) leaves results near zero where
    # ulps are meaningless; there the fp32 error bound 2^-24*|x| applies
    assert within_ulp_or_abs(xd.cpu(), x_new, 1, 1e-6) and (xd.cpu() != x_new).float().mean() < 1e-3
    torch.testing.assert_close(y, ops.rmsnorm(xd.cpu(), w, 1e-6), atol=.016, rtol=.008)


# ---------------------------------------------------------------- kv store --

@pytest.mark.parametrize("capacity", [8, 4096])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@torch.inference_mode()
def test_kv_write_bitwise_strided_inactive_and_graph(capacity, dtype):
    """Reference test_fused_kv_write.py:7-46."""
    cfg = ModelConfig(num_key_value_heads=3, hidden_size=21, num_attention_heads=3, num_hidden_layers=2)
    cache = KVCache(cfg, 3, capacity, DEV, dtype)
    cache.k.normal_()
    cache.v.normal_()
    k = torch.randn(3, 3, 1, 28, device=DEV, dtype=dtype)[..., ::4]
    v = torch.randn(3, 3, 1, 42, device=DEV, dtype=dtype)[..., 1::6]
    pos = torch.tensor([0, capacity + 10, capacity - 1], device=DEV)
    active = torch.tensor([True, False, True], device=DEV)
    k[1].fill_(float("nan"))
    v[1].fill_(float("nan"))
    expected_k, expected_v = cache.k.clone(), cache.v.clone()
    for slot, p in ((0, 0), (2, capacity - 1)):
        expected_k[1, slot, :, p] = k[slot, :, 0]
        expected_v[1, slot, :, p] = v[slot, :, 0]
    cache.write(1, k, v, pos, active)
    torch.cuda.synchronize()
    assert torch.equal(cache.k, expected_k) and torch.equal(cache.v, expected_v)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cache.write(1, k, v, pos, active)
    for replay in range(3):
        pos.copy_(torch.tensor([1 + replay, 2 + replay, capacity + 99], device=DEV))
        active.copy_(torch.tensor([True, True, False], device=DEV))
        k.normal_()
        v.normal_()
        for slot in (0, 1):
            expected_k[1, slot, :, 1 + replay + slot] = k[slot, :, 0]
            expected_v[1, slot, :, 1 + replay + slot] = v[slot, :, 0]
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(cache.k, expected_k) and torch.equal(cache.v, expected_v)


# -------------------------------------------------------------------- rope --

@torch.inference_mode()
def test_rope_bitwise_on_packed_views():
    """Rotation equals the torch formula of model.py:66-67 bit for bit on
    strided views of a packed QKV buffer (vLLM entry, model.py:63-64)."""
    t, hq, hkv, d = 37, 24, 8, 64
    cos_sin, cos, sin = ops.rope_tables(1e4, d, 4096, torch.bfloat16)
    qkv = bf((t, (hq + 2 * hkv) * d), 1.0, 6)
    pos = torch.randint(0, 4096, (t,))
    dev = qkv.to(DEV)
    q = dev[:, :hq * d].view(t, hq, d)
    k = dev[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    rope.rotary_embedding(pos.to(DEV), q, k, d, cos_sin.to(DEV))
    eq = ops.rope(qkv[:, :hq * d].view(t, hq, d), cos, sin, pos)
    ek = ops.rope(qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d), cos, sin, pos)
    assert torch.equal(q.cpu(), eq) and torch.equal(k.cpu(), ek)
    assert torch.equal(dev[:, (hq + hkv) * d:].cpu(), qkv[:, (hq + hkv) * d:])  # v untouched


@pytest.mark.parametrize("write_k", [False, True])
@torch.inference_mode()
def test_rope_kv_write_stores_rotated_k_and_v(write_k):
    t, hq, hkv, d, cap = 9, 6, 2, 64, 32
    cfg = ModelConfig(num_key_value_heads=hkv, hidden_size=hq * d, num_attention_heads=hq, num_hidden_layers=2)
    cache = KVCache(cfg, 4, cap, DEV, torch.bfloat16)
    cache.k.normal_()
    cache.v.normal_()
    before_k, before_v = cache.k.cpu(), cache.v.cpu()
    cos_sin, cos, sin = ops.rope_tables(1e4, d, cap, torch.bfloat16)
    qkv = bf((t, (hq + 2 * hkv) * d), 1.0, 7)
    pos = torch.tensor([0, 1, 2, 31, 5, 40, 7, 3, 4])
    active = torch.tensor([True, True, True, True, False, True, True, True, True])
    slots = torch.tensor([0, 0, 0, 3, 1, 2, 9, 1, 1])  # slot 9 and position 40 out of range: skipped
    dev = qkv.to(DEV)
    q = dev[:, :hq * d].view(t, hq, d)
    k = dev[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    v = dev[:, (hq + hkv) * d:].view(t, hkv, d)
    rope.rope_kv_write(q, k, v, pos.to(DEV), active.to(DEV), cos_sin.to(DEV), cache, 1, slots.to(DEV), write_k)
    rk = ops.rope(qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d), cos, sin, pos.clamp(max=cap - 1))
    rv = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    ek, ev = ops.kv_store(before_k[1], before_v[1], rk, rv, pos, active, slots)
    assert torch.equal(cache.k[1].cpu(), ek) and torch.equal(cache.v[1].cpu(), ev)
    assert torch.equal(cache.k[0].cpu(), before_k[0])
    assert torch.equal(q.cpu()[:5], ops.rope(qkv[:5, :hq * d].view(5, hq, d), cos, sin, pos[:5]))
    if write_k:
        assert torch.equal(k.cpu()[:5], rk[:5])
    else:
        assert torch.equal(k.cpu(), qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d))


# ------------------------------------------------------------------ router --

@pytest.mark.parametrize("m,h,e,k", [(16, 1024, 32, 8), (64, 1536, 40, 8), (4096, 1536, 40, 8), (7, 256, 8, 2),
                                      (32, 1024, 128, 8), (16, 4096, 256, 8), (9, 3072, 60, 6), (5, 1280, 40, 8)])
@torch.inference_mode()
def test_router_ids_bit_exact_given_logits(m, h, e, k):
    z = bf((m, h), 1.0, 10 + m)
    wr = bf((e, h), 0.02 * 8, 20 + m)
    logits = torch.empty(m, e, device=DEV, dtype=torch.bfloat16)
    weights, ids = router.route(z.to(DEV), wr.to(DEV), k, logits_out=logits)
    logits = logits.cpu()
    cpu_logits = torch.nn.functional.linear(z, wr)
    # GEMV accumulation order differs from the CPU BLAS: a logit may move by
    # one bf16 ulp, rarely.
    assert within_ulp_or_abs(logits, cpu_logits, 1, 2e-3)
    assert (logits != cpu_logits).float().mean() < 0.02
    ew, eids = ops.route(logits, k)
    assert torch.equal(ids.cpu(), eids)
    torch.testing.assert_close(weights.cpu(), ew, rtol=2e-6, atol=1e-7)
    # end to end: every id mismatch must come with a logit difference
    _, cpu_ids = ops.route(cpu_logits, k)
    bad = (cpu_ids != ids.cpu()).any(-1)
    assert bool(((logits != cpu_logits).any(-1) | ~bad).all())


@pytest.mark.parametrize("renormalize", [True, False])
@torch.inference_mode()
def test_topk_softmax_ties_go_to_lower_id(renormalize):
    g = torch.Generator().manual_seed(3)
    logits = torch.randint(-3, 4, (300, 40), generator=g).to(torch.bfloat16)
    weights, ids, idx = router.fused_topk(None, logits.to(DEV), 8, renormalize=renormalize)
    ew, eids = ops.route(logits, 8, renormalize=renormalize)
    assert torch.equal(ids.cpu(), eids)
    torch.testing.assert_close(weights.cpu(), ew, rtol=2e-6, atol=1e-7)
    assert torch.equal(idx.cpu().flatten(), torch.arange(300 * 8, dtype=torch.int32))


# ------------------------------------------------------------- permutation --

@pytest.mark.parametrize("m,k,e,first,local", [(64, 8, 40, 0, 40), (16, 8, 32, 0, 32), (4096, 8, 40, 0, 40),
                                                (64, 8, 40, 10, 5), (1, 1, 4, 0, 4), (50000, 8, 40, 0, 40)])
@torch.inference_mode()
def test_moe_align_bit_exact(m, k, e, first, local):
    g = torch.Generator().manual_seed(m + first)
    ids = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(m)]).to(torch.int32) if m < 5000 else \
        torch.randint(0, e, (m, k), generator=g, dtype=torch.int32)
    offsets, order, inverse = experts.moe_align(ids.to(DEV), local, first)
    eo, eord, einv = ops.permutation(ids, local, first)
    assert offsets.cpu().tolist() == eo.tolist()
    assert torch.equal(order.cpu().long(), eord)
    assert torch.equal(inverse.cpu().long(), einv)


@torch.inference_mode()
def test_moe_align_skewed():
    g = torch.Generator().manual_seed(9)
    hot = torch.randint(0, 4, (20000, 8), generator=g)
    cold = torch.randint(0, 40, (20000, 8), generator=g)
    ids = torch.where(torch.rand(20000, 8, generator=g) < 0.5, hot, cold).to(torch.int32)
    offsets, order, _ = experts.moe_align(ids.to(DEV), 40)
    eo, eord, _ = ops.permutation(ids, 40)
    assert offsets.cpu().tolist() == eo.tolist() and torch.equal(order.cpu().long(), eord)


# ----------------------------------------------------------------- experts --

def _moe_inputs(m, h, i, e, k, seed):
    x = bf((m, h), 1.0, seed)
    w1 = bf((e, 2 * i, h), 0.02, seed + 1)
    w2 = bf((e, h, i), 0.02, seed + 2)
    wr = bf((e, h), 0.02, seed + 3)
    weights, ids = ops.route(torch.nn.functional.linear(x, wr), k)
    return x, w1, w2, weights, ids


@pytest.mark.parametrize("m,h,i,e,k", [(16, 1024, 512, 32, 8), (64, 1536, 512, 40, 8), (5, 1536, 512, 40, 8),
                                       (300, 1024, 512, 32, 8), (64, 256, 128, 8, 2)])
@torch.inference_mode()
def test_expert_stages_match_oracle(m, h, i, e, k):
    x, w1, w2, weights, ids = _moe_inputs(m, h, i, e, k, 100 + m)
    offsets, order, _ = experts.moe_align(ids.to(DEV), e)
    act = experts.gate_up(x.to(DEV), w1.to(DEV), offsets, order, k).cpu()
    flat = ids.flatten().long()
    exp_act = torch.empty_like(act)
    for r in range(flat.numel()):
        gate, up = torch.nn.functional.linear(x[r // k][None], w1[flat[r]]).chunk(2, -1)
        exp_act[r] = (torch.nn.functional.silu(gate) * up)[0]
    assert rel_l2(act, exp_act) < 5e-3
    y = experts.down(act.to(DEV), w2.to(DEV), offsets, order).cpu()
    ey = ops.expert_routes(x, ids, w1, w2)
    assert rel_l2(y, ey) < 1e-2


@pytest.mark.parametrize("m,h,i,e,k", [(16, 1024, 512, 32, 8), (64, 1536, 512, 40, 8), (1, 1536, 512, 40, 8),
                                       (512, 1536, 512, 40, 8)])
@torch.inference_mode()
def test_fused_experts_match_oracle(m, h, i, e, k):
    x, w1, w2, weights, ids = _moe_inputs(m, h, i, e, k, 200 + m)
    out = experts.fused_experts(x.to(DEV), w1.to(DEV), w2.to(DEV), weights.to(DEV), ids.to(DEV)).cpu()
    expected = ops.fused_moe(x, ids, weights, w1, w2)
    assert rel_l2(out, expected) < 1e-2          # north-star bar 2e-2
    reference = ops.reference_experts(x, ids, weights.to(torch.bfloat16).float(), w1, w2, singleton=True)
    assert rel_l2(out, reference) < 2e-2          # the reference CPU path


@pytest.mark.parametrize("m", [64, 600])
@torch.inference_mode()
def test_fused_experts_repeated_and_out_of_range_ids(m):
    """Expert ids are device data and are not validated at the call. A token
    that lists an expert several times gets every route computed and
    combined (litemoe/ops.py:34-55 does the same); at m=64 (scan path) every
    token lists expert 3 five times, so expert 3 has about 270 routes:
    more than the call's 64 tokens and more than 256 (a per-expert route
    list sized by the token count would drop the rest). Ids outside
    [0, E) add nothing: compared with the oracle on the same routes with
    those scales set to zero. m=600 takes the aligned-block path."""
    h, i, e, k = 1536, 512, 40, 8
    x, w1, w2, weights, ids = _moe_inputs(m, h, i, e, k, 300 + m)
    ids = ids.clone()
    ids[:, 3:] = 3                       # five repeats of expert 3 in every token
    ids[::7] = 11                        # some tokens route all eight branches to 11
    bad = torch.zeros_like(ids, dtype=torch.bool)
    bad[1::5, 0] = True
    bad[2::9, 2] = True
    ids_dev = torch.where(bad, torch.where(torch.arange(m)[:, None] % 2 == 0, e, -1), ids)
    out = experts.fused_experts(x.to(DEV), w1.to(DEV), w2.to(DEV), weights.to(DEV),
                                ids_dev.int().to(DEV)).cpu()
    scales = torch.where(bad, 0.0, weights)
    safe_ids = torch.where(bad, 0, ids)
    expected = ops.fused_moe(x, safe_ids.int(), scales, w1, w2)
    assert rel_l2(out, expected) < 1e-2
    reference = ops.reference_experts(x, safe_ids, scales.to(torch.bfloat16).float(), w1, w2, singleton=True)
    assert rel_l2(out, reference) < 2e-2
    per_row = (out.float() - expected.float()).norm(dim=1) / expected.float().norm(dim=1).clamp_min(1e-6)
    assert float(per_row.max()) < 5e-2


@torch.inference_mode()
def test_fused_experts_block_rows_do_not_change_results():
    x, w1, w2, weights, ids = _moe_inputs(200, 1024, 512, 8, 2, 7)
    args = [t.to(DEV) for t in (x, w1, w2, weights, ids)]
    base = experts.fused_experts(*args, block_rows=0)
    for bm in (16, 48, 256):
        assert torch.equal(experts.fused_experts(*args, block_rows=bm), base)


@pytest.mark.parametrize("m,h,i,e,k,skew", [(2048, 256, 128, 64, 8, False), (2048, 256, 128, 64, 8, True),
                                            (1100, 512, 256, 20, 4, False),
                                            (8192, 256, 128, 16, 8, False), (8192, 256, 128, 16, 8, True)])
@torch.inference_mode()
def test_prefill_expert_gemm_and_chunked_align_match_oracle(m, h, i, e, k, skew):
    """Prefill-sized route counts (>= 4096 routes): lm_moe_routes takes the
    LDS-tiled MFMA GEMMs (128-route blocks; 256-route blocks from 1024 routes
    per expert, the m=8192 cases), and above 8192 routes the chunked
    three-launch align. Route outputs against the oracle's per-route expert
    math; skew puts most routes on two experts and leaves some empty."""
    x, w1, w2, _, ids = _moe_inputs(m, h, i, e, k, 700 + m)
    if skew:
        g = torch.Generator().manual_seed(m)
        p = torch.full((e,), 0.1 / (e - 8))
        p[:2] = 0.45
        p[-6:] = 0.0  # experts with no route at all
        ids = torch.stack([torch.multinomial(p, k, replacement=False, generator=g) for _ in range(m)]).int()
    y = experts.moe_routes(x.to(DEV), w1.to(DEV), w2.to(DEV), ids.to(DEV)).cpu()
    exp = ops.expert_routes(x, ids, w1, w2)
    assert rel_l2(y, exp) < 1e-2
    # every route row written: no NaN/garbage rows, each row close on its own
    per_row = (y.float() - exp.float()).norm(dim=1) / exp.float().norm(dim=1).clamp_min(1e-6)
    assert float(per_row.max()) < 5e-2


@pytest.mark.parametrize("m,e", [(50000, 40), (13000, 96)])
@torch.inference_mode()
def test_chunked_align_long_and_wide_scans_match_oracle(m, e):
    """The chunked align's scan beyond 384 chunks of 1024 routes (400,000
    routes: its looped form) and with more than 64 expert keys (97: two key
    groups), under the 256-route expert GEMMs: the routes of 256 sampled
    tokens against the oracle's per-route expert math (a wrong permutation
    sends a route to another expert's weights or its row to another route)."""
    h, i, k = 256, 128, 8
    g = torch.Generator().manual_seed(m + e)
    x = torch.randn(m, h, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(e, 2 * i, h, generator=g) * 0.05).to(torch.bfloat16)
    w2 = (torch.randn(e, h, i, generator=g) * 0.05).to(torch.bfloat16)
    ids = torch.rand(m, e, generator=g).argsort(dim=1)[:, :k].to(torch.int32)
    y = experts.moe_routes(x.to(DEV), w1.to(DEV), w2.to(DEV), ids.to(DEV)).cpu()
    sample = torch.randperm(m, generator=g)[:256]
    exp = ops.expert_routes(x[sample], ids[sample], w1, w2)
    got = y.view(m, k, h)[sample].reshape(-1, h)
    assert rel_l2(got, exp) < 1e-2
    per_row = (got.float() - exp.float()).norm(dim=1) / exp.float().norm(dim=1).clamp_min(1e-6)
    assert float(per_row.max()) < 5e-2


@torch.inference_mode()
def test_prefill_expert_gemm_close_to_block_kernels():
    """The GEMM path (block_rows=0) against the per-tile block kernels
    (explicit block_rows) on the 3B shape: same math, different fp32
    accumulation order."""
    x, w1, w2, _, ids = _moe_inputs(1024, 1536, 512, 40, 8, 77)
    args = [t.to(DEV) for t in (x, w1, w2)]
    gemm = experts.moe_routes(*args, ids.to(DEV))
    block = experts.moe_routes(*args, ids.to(DEV), block_rows=128)
    assert rel_l2(gemm.cpu(), block.cpu()) < 2e-3
    again = experts.moe_routes(*args, ids.to(DEV))
    assert torch.equal(gemm, again)  # deterministic


# ------------------------------------------------------------------ finish --

@pytest.mark.parametrize("batch,topk,hidden,rank,world,remap", [
    (1, 8, 1536, 0, 1, False), (8, 8, 2048, 0, 1, True), (32, 8, 65, 1, 2, False),
    (8, 3, 129, 0, 2, True), (1, 1, 65, 0, 1, False)])
@torch.inference_mode()
def test_finish_bit_exact_mask_order_and_graph(batch, topk, hidden, rank, world, remap):
    """Reference test_moe_finish.py:20-71 cases; bit-exact vs the oracle."""
    torch.manual_seed(29)
    count = 8

    def make():
        ids = torch.stack([torch.randperm(count * world)[:topk] for _ in range(batch)]).int()
        order = ids.flatten().argsort()
        y = torch.randn(batch * topk, hidden).to(torch.bfloat16)
        scales = torch.softmax(torch.randn(batch, topk), -1)
        if batch > 1:
            scales[-1] = 0
        selected = ids.flatten()[order].long() - rank * count
        y[(selected < 0) | (selected >= count)] = float("nan")
        return ids, order, y, scales

    logical = torch.randperm(count * world) if remap else None
    ids, order, y, scales = make()
    d = [t.to(DEV) for t in (ids, order, y, scales)]
    lg = logical.to(DEV) if remap else None
    out = torch.empty(batch, hidden, device=DEV, dtype=torch.bfloat16)

    def check():
        inverse = torch.empty_like(order)
        inverse[order] = torch.arange(order.numel())
        expected = ops.finish(y, ids, scales, rank, count, logical, inverse=inverse)
        got = out.cpu()
        assert torch.isfinite(got).all() and torch.equal(got, expected)
        if batch > 1:
            assert torch.count_nonzero(got[-1]) == 0

    moe_finish.finish(d[2], d[0], d[1], d[3], out, rank, count, lg)
    check()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        moe_finish.finish(d[2], d[0], d[1], d[3], out, rank, count, lg)
    for _ in range(2):
        ids, order, y, scales = make()
        for dst, src in zip(d, (ids, order, y, scales)):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        check()


@torch.inference_mode()
def test_finish_never_reads_all_nonlocal_nan_rows():
    ids = torch.tensor([[0, 1, 2]], device=DEV, dtype=torch.int32)
    y = torch.full((3, 65), float("nan"), device=DEV, dtype=torch.bfloat16)
    out = torch.full((1, 65), float("nan"), device=DEV, dtype=torch.bfloat16)
    moe_finish.finish(y, ids, ids.flatten().long(), torch.ones(1, 3, device=DEV), out, 1, 4)
    assert torch.equal(out, torch.zeros_like(out))


# --------------------------------------------------------------- attention --

@pytest.mark.parametrize("b,hq,hkv,cap,low,high,splits", [
    (64, 24, 8, 2048, 1, 1280, None), (32, 16, 8, 1024, 1, 640, 1), (5, 24, 8, 256, 1, 256, 3),
    (128, 24, 8, 4096, 1024, 4096, None),
    # the other query-group sizes the kernel is built for (q heads per kv head 1, 4, 6, 8)
    (4, 8, 8, 256, 1, 256, None), (6, 32, 8, 512, 1, 512, None), (3, 48, 8, 300, 1, 300, 2),
    (5, 64, 8, 512, 1, 512, None)])
@torch.inference_mode()
def test_flash_decode_matches_oracle(b, hq, hkv, cap, low, high, splits):
    g = torch.Generator().manual_seed(b + cap)
    q = torch.randn(b, hq, 64, generator=g).to(torch.bfloat16)
    kc = torch.randn(b, hkv, cap, 64, generator=g).to(torch.bfloat16)
    vc = torch.randn(b, hkv, cap, 64, generator=g).to(torch.bfloat16)
    used = torch.randint(low, high + 1, (b,), generator=g, dtype=torch.int32)
    used[0] = 1
    fd = flash_decode.FlashDecode(b, hkv, hq // hkv, cap, DEV, maximum=high, num_splits=splits)
    got = fd(q.to(DEV)[:, :, None], kc.to(DEV), vc.to(DEV), None, None, 0.125, used=used.to(DEV))[:, :, 0].cpu()
    rows = list(range(min(b, 24))) + ([b - 1] if b > 24 else [])
    exp = ops.decode_attention(q[rows], kc[rows], vc[rows], used[rows], 0.125)
    torch.testing.assert_close(got[rows], exp, atol=.004, rtol=.03)  # reference test_flash_decode.py:53-56
    assert rel_l2(got[rows], exp) < 5e-3


@pytest.mark.parametrize("pattern", ["ramp", "sawtooth", "wide", "falling"])
@pytest.mark.parametrize("splits,hq", [(None, 24), (3, 24), (None, 8), (2, 64)])
@torch.inference_mode()
def test_flash_decode_score_drift_matches_oracle(pattern, splits, hq):
    """Scores that move the running maximum many times, by steps below and
    above the kernel's slack of 8 (log2 units) before it rescales: a ramp of
    0.06 per key up to ~60, a sawtooth of +5 / +11 jumps, a spread of std 20,
    and a falling ramp (the maximum at the first key)."""
    b, hkv, cap = 6, 8, 1024
    g = torch.Generator().manual_seed(11)
    q = torch.randn(b, hq, 64, generator=g)
    j = torch.arange(cap, dtype=torch.float32)
    if pattern == "ramp":
        t = 0.06 * j - 10
    elif pattern == "sawtooth":
        t = torch.where((j // 16) % 2 == 0, 5.0, 11.0) * (j // 16 % 5) + 0.01 * j
    elif pattern == "wide":
        t = 20 * torch.randn(cap, generator=g)
    else:
        t = 30 - 0.05 * j
    # k of kv head h lies along q of its group's first q head: scale * q.k = t (natural log units)
    lead = q[:, ::hq // hkv]  # [b, hkv, 64]
    kc = t[None, None, :, None] * lead[:, :, None, :] / (0.125 * lead.square().sum(-1))[:, :, None, None]
    kc = (kc + 0.05 * torch.randn(b, hkv, cap, 64, generator=g)).to(torch.bfloat16)
    q = q.to(torch.bfloat16)
    vc = torch.randn(b, hkv, cap, 64, generator=g).to(torch.bfloat16)
    used = torch.tensor([1024, 1000, 777, 300, 129, 17], dtype=torch.int32)
    fd = flash_decode.FlashDecode(b, hkv, hq // hkv, cap, DEV, maximum=cap, num_splits=splits)
    got = fd(q.to(DEV)[:, :, None], kc.to(DEV), vc.to(DEV), None, None, 0.125, used=used.to(DEV))[:, :, 0].cpu()
    exp = ops.decode_attention(q, kc, vc, used, 0.125)
    assert torch.isfinite(got.float()).all()
    torch.testing.assert_close(got, exp, atol=.004, rtol=.03)
    assert rel_l2(got, exp) < 5e-3


@torch.inference_mode()
def test_flash_decode_lengths_active_and_empty_rows():
    b, hq, hkv, cap = 4, 6, 2, 64
    q = torch.randn(b, hq, 1, 64, device=DEV).to(torch.bfloat16)
    kc = torch.randn(b, hkv, cap, 64, device=DEV).to(torch.bfloat16)
    vc = torch.randn(b, hkv, cap, 64, device=DEV).to(torch.bfloat16)
    fd = flash_decode.FlashDecode(b, hkv, hq // hkv, cap, DEV, maximum=63, num_splits=4)
    lengths = torch.tensor([62, 999, 0, 10], device=DEV)
    active = torch.tensor([True, False, True, True], device=DEV)
    got = fd(q, kc, vc, lengths, active, 0.125)[:, :, 0].cpu()
    used = torch.tensor([63, 1, 1, 11], dtype=torch.int32)
    exp = ops.decode_attention(q[:, :, 0].cpu(), kc.cpu(), vc.cpu(), used, 0.125)
    torch.testing.assert_close(got, exp, atol=.004, rtol=.03)
    zero = fd(q, kc, vc, None, None, 0.125, used=torch.zeros(b, dtype=torch.int32, device=DEV))
    assert torch.equal(zero, torch.zeros_like(zero))


@pytest.mark.parametrize("lengths", [[2, 7], [1, 17, 64, 65, 130, 300], [2048, 64, 700]])
@torch.inference_mode()
def test_prefill_attention_matches_oracle_and_isolates_sequences(lengths):
    t = sum(lengths)
    g = torch.Generator().manual_seed(t)
    hq, hkv = 24, 8
    q = torch.randn(t, hq, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(t, hkv, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(t, hkv, 64, generator=g).to(torch.bfloat16)
    cu = torch.tensor([0] + lengths).cumsum(0).to(torch.int32)
    got = packed.varlen_attention(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), max(lengths), 0.125).cpu()
    exp = ops.varlen_attention(q, k, v, cu, 0.125)
    torch.testing.assert_close(got, exp, atol=.016, rtol=.016)  # reference test_packed_prefill.py:40
    assert rel_l2(got, exp) < 1e-2
    # Perturb token 1: outputs of every other sequence, and of its own
    # sequence before it (causal), stay bit-identical.
    k2, v2 = k.clone(), v.clone()
    k2[1] += 4
    v2[1] += 4
    changed = packed.varlen_attention(q.to(DEV), k2.to(DEV), v2.to(DEV), cu.to(DEV), max(lengths), 0.125).cpu()
    seq = int((cu[1:] <= 1).sum())
    start, end = int(cu[seq]), int(cu[seq + 1])
    assert torch.equal(changed[:start], got[:start]) and torch.equal(changed[end:], got[end:])
    assert torch.equal(changed[start:1], got[start:1])
    assert not torch.equal(changed[1:end], got[1:end])


@pytest.mark.parametrize("lengths,hq,hkv,causal", [
    ([1, 17, 64, 65, 130, 300], 24, 8, False),   # non-causal: every key of the sequence
    ([3, 0, 129, 5], 16, 8, True),               # an empty sequence inside the pack
    ([250, 1, 128], 8, 8, True),                 # one q head per kv head
    ([257, 31], 32, 4, False)])
@torch.inference_mode()
def test_prefill_attention_modes_and_head_ratios(lengths, hq, hkv, causal):
    t = sum(lengths)
    g = torch.Generator().manual_seed(t + hq)
    q = torch.randn(t, hq, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(t, hkv, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(t, hkv, 64, generator=g).to(torch.bfloat16)
    cu = torch.tensor([0] + lengths).cumsum(0).to(torch.int32)
    got = packed.varlen_attention(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), max(lengths), 0.125,
                                  causal=causal).cpu()
    exp = ops.varlen_attention(q, k, v, cu, 0.125, causal=causal)
    torch.testing.assert_close(got, exp, atol=.016, rtol=.016)
    assert rel_l2(got, exp) < 1e-2


# ----------------------------------------------------------- fused decode ops --

@pytest.mark.parametrize("m", [1, 16, 64, 256, 257])
@torch.inference_mode()
def test_moe_routes_scan_path_equals_block_path(m):
    """The decode path (each expert collects its own routes, m <= 256) and the
    aligned-block path give bit-identical route outputs."""
    x, w1, w2, weights, ids = _moe_inputs(m, 1536, 512, 40, 8, 300 + m)
    args = [t.to(DEV) for t in (x, w1, w2)]
    scan = experts.moe_routes(*args, ids.to(DEV))
    blocks = experts.moe_routes(*args, ids.to(DEV), block_rows=16)
    assert torch.equal(scan, blocks)
    if m <= 16:
        assert rel_l2(scan.cpu(), ops.expert_routes(x, ids, w1, w2)) < 1e-2


@pytest.mark.parametrize("m,e,hot", [(64, 40, False), (64, 40, True), (60, 36, False), (64, 33, True),
                                     (48, 40, True), (64, 40, None)])
@torch.inference_mode()
def test_gate_up_scan_path_equals_block_path(m, e, hot):
    """The decode gate/up (each expert's workgroups collect its routes from
    topk_ids) equals the aligned-block path bit for bit, including experts
    with more than 16 routes (hot: four experts in every token's top-8, up to
    64 routes each) and experts with none (None: only 8 experts used)."""
    h, i, k = 1536, 512, 8
    x, w1, _, _, ids = _moe_inputs(m, h, i, e, k, 500 + m + e)
    g = torch.Generator().manual_seed(m + e)
    if hot:  # distinct ids per token: 0..3, then four of 4..e-1
        ids = torch.stack([torch.cat([torch.arange(4), 4 + torch.randperm(e - 4, generator=g)[:4]])
                           for _ in range(m)]).int()
    elif hot is None:
        ids = torch.stack([torch.randperm(8, generator=g) for _ in range(m)]).int()
    xd, w1d, idsd = x.to(DEV), w1.to(DEV), ids.to(DEV)
    scan = experts.gate_up(xd, w1d, None, None, k, topk_ids=idsd)
    offsets, order, _ = experts.moe_align(idsd, e)
    blocks = experts.gate_up(xd, w1d, offsets, order, k, block_rows=16)
    assert torch.equal(scan, blocks)


@torch.inference_mode()
def test_finish_add_rmsnorm_equals_unfused():
    m, h, k, e = 64, 1536, 8, 40
    g = torch.Generator().manual_seed(12)
    y = torch.randn(m * k, h, generator=g).to(torch.bfloat16).to(DEV)
    ids = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(m)]).int().to(DEV)
    scales = torch.softmax(torch.randn(m, k, generator=g), -1).to(DEV)
    x = torch.randn(m, h, generator=g).to(torch.bfloat16).to(DEV)
    w = (1 + 0.2 * torch.randn(h, generator=g)).to(torch.bfloat16).to(DEV)
    x1, x2 = x.clone(), x.clone()
    z1 = experts.finish_add_rmsnorm(y, ids, scales, x1, 0.22, w, 1e-6)
    out = torch.empty(m, h, device=DEV, dtype=torch.bfloat16)
    moe_finish.finish(y, ids, torch.arange(m * k, device=DEV), scales, out, 0, e)
    z2 = norm.add_rmsnorm(x2, out, 0.22, w, 1e-6)
    assert torch.equal(x1, x2) and torch.equal(z1, z2)


@pytest.mark.parametrize("h", [1536, 1280])
@pytest.mark.parametrize("with_residual", [False, True])
@torch.inference_mode()
def test_add_rmsnorm_route_equals_unfused(with_residual, h):
    m, e, k = 64, 40, 8
    g = torch.Generator().manual_seed(13)
    x = torch.randn(m, h, generator=g).to(torch.bfloat16).to(DEV)
    a = torch.randn(m, h, generator=g).to(torch.bfloat16).to(DEV) if with_residual else None
    w = (1 + 0.2 * torch.randn(h, generator=g)).to(torch.bfloat16).to(DEV)
    wr = (0.02 * torch.randn(e, h, generator=g)).to(torch.bfloat16).to(DEV)
    x1, x2 = x.clone(), x.clone()
    logits1 = torch.empty(m, e, device=DEV, dtype=torch.bfloat16)
    w1_, i1, z1 = router.add_rmsnorm_route(x1, a, 0.22, w, 1e-6, wr, k, logits_out=logits1)
    z2 = norm.add_rmsnorm(x2, a, 0.22, w, 1e-6)
    logits2 = torch.empty(m, e, device=DEV, dtype=torch.bfloat16)
    w2_, i2 = router.route(z2, wr, k, logits_out=logits2)
    assert torch.equal(x1, x2) and torch.equal(z1, z2) and torch.equal(logits1, logits2)
    assert torch.equal(i1, i2) and torch.equal(w1_, w2_)


def per_token_logits(z, wr, k, chunk=256):
    """Router logits from the per-token GEMV kernels (calls below the batched
    kernel's token count)."""
    out = torch.empty(z.shape[0], wr.shape[0], device=DEV, dtype=torch.bfloat16)
    for c in range(0, z.shape[0], chunk):
        router.route(z[c:c + chunk], wr, k, logits_out=out[c:c + chunk])
    return out


@pytest.mark.parametrize("m,h,e,k,with_residual", [(4103, 1536, 40, 8, True), (4096, 1536, 40, 8, False),
                                                   (4111, 1024, 32, 4, True), (4100, 4096, 64, 8, True),
                                                   (4096, 3072, 60, 6, True), (4104, 512, 20, 2, True),
                                                   (4097, 2048, 48, 8, True), (4100, 1536, 64, 8, True)])
@torch.inference_mode()
def test_batched_add_rmsnorm_route(m, h, e, k, with_residual):
    """Prefill-sized calls take the batched MFMA router (16 tokens per wave,
    a tail below 16 on the per-token kernel): x and z bitwise the unfused
    norm's, logits within one bf16 ulp of the GEMV kernels' and of the CPU
    product, ids exact given the kernel's own logits."""
    g = torch.Generator().manual_seed(m + h)
    x = torch.randn(m, h, generator=g).to(torch.bfloat16).to(DEV)
    a = torch.randn(m, h, generator=g).to(torch.bfloat16).to(DEV) if with_residual else None
    w = (1 + 0.2 * torch.randn(h, generator=g)).to(torch.bfloat16).to(DEV)
    wr = (0.02 * torch.randn(e, h, generator=g)).to(torch.bfloat16).to(DEV)
    x1, x2 = x.clone(), x.clone()
    logits1 = torch.empty(m, e, device=DEV, dtype=torch.bfloat16)
    w1_, i1, z1 = router.add_rmsnorm_route(x1, a, 0.22, w, 1e-6, wr, k, logits_out=logits1)
    z2 = norm.add_rmsnorm(x2, a, 0.22, w, 1e-6)
    assert torch.equal(x1, x2) and torch.equal(z1, z2)
    logits2 = per_token_logits(z2, wr, k)
    tail = m % 16
    if tail:
        assert torch.equal(logits1[m - tail:], logits2[m - tail:])
    assert within_ulp_or_abs(logits1, logits2, 1, 2e-3)
    assert (logits1 != logits2).float().mean() < 0.02
    cpu_logits = torch.nn.functional.linear(z1.cpu(), wr.cpu())
    assert within_ulp_or_abs(logits1.cpu(), cpu_logits, 1, 2e-3)
    ew, eids = ops.route(logits1.cpu(), k)
    assert torch.equal(i1.cpu(), eids)
    torch.testing.assert_close(w1_.cpu(), ew, rtol=2e-6, atol=1e-7)
    # without logits_out the same selection
    x3 = x.clone()
    w3_, i3, z3 = router.add_rmsnorm_route(x3, a, 0.22, w, 1e-6, wr, k)
    assert torch.equal(i3, i1) and torch.equal(w3_, w1_) and torch.equal(z3, z1)


@pytest.mark.parametrize("renormalize", [True, False])
@torch.inference_mode()
def test_batched_route_without_norm(renormalize):
    m, h, e, k = 4099, 1536, 40, 8
    z = bf((m, h), 1.0, 77).to(DEV)
    wr = bf((e, h), 0.02, 78).to(DEV)
    logits = torch.empty(m, e, device=DEV, dtype=torch.bfloat16)
    weights, ids = router.route(z, wr, k, renormalize=renormalize, logits_out=logits)
    assert within_ulp_or_abs(logits, per_token_logits(z, wr, k), 1, 2e-3)
    ew, eids = ops.route(logits.cpu(), k, renormalize=renormalize)
    assert torch.equal(ids.cpu(), eids)
    torch.testing.assert_close(weights.cpu(), ew, rtol=2e-6, atol=1e-7)


# ----------------------------------------------------- packed expert weights --

@torch.inference_mode()
def test_expert_pack_layout():
    """lm_expert_pack's chunk (tile, k, lane) of each matrix M [rows, K] is
    M[16*tile + lane%16, 32*k + 8*(lane//16):+8] (w1 as [E*2I, H], w2 as [E*H, I])."""
    e, h, i = 3, 256, 128
    w1, w2 = bf((e, 2 * i, h), 1.0, 1), bf((e, h, i), 1.0, 2)
    p1, p2 = experts.pack_expert_weights(w1.to(DEV), w2.to(DEV))

    def expect(m, rows, kk):
        return m.reshape(rows // 16, 16, kk // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(-1)

    assert torch.equal(p1.cpu().reshape(-1), expect(w1, e * 2 * i, h))
    assert torch.equal(p2.cpu().reshape(-1), expect(w2, e * h, i))


@pytest.mark.parametrize("m,h,i,e,k,block_rows", [
    (64, 1536, 512, 40, 8, 0),      # decode scan path (Granite-3B decode)
    (1, 1536, 512, 40, 8, 0),
    (32, 1024, 512, 32, 8, 0),      # Granite-1B decode
    (300, 1024, 512, 32, 8, 0),     # block path (more than 256 tokens)
    (64, 1536, 512, 40, 8, 16),     # block path forced
    (640, 1024, 512, 32, 8, 0),     # prefill expert GEMM (>= 4096 routes)
    (64, 256, 128, 8, 2, 0),
])
@torch.inference_mode()
def test_packed_weights_give_the_same_bits(m, h, i, e, k, block_rows):
    """Every expert kernel reads the fragment layout to the same bits as the
    checkpoint layout: the route outputs, the two stages and the fused call."""
    x, w1, w2, weights, ids = _moe_inputs(m, h, i, e, k, 900 + m + h)
    xd, w1d, w2d, idsd, wd = (t.to(DEV) for t in (x, w1, w2, ids, weights))
    p1, p2 = experts.pack_expert_weights(w1d, w2d)
    ref = experts.moe_routes(xd, w1d, w2d, idsd, block_rows=block_rows)
    got = experts.moe_routes(xd, p1, p2, idsd, block_rows=block_rows, packed=True)
    assert torch.equal(got, ref)
    out_ref = experts.fused_experts(xd, w1d, w2d, wd, idsd, block_rows=block_rows)
    out = experts.fused_experts(xd, p1, p2, wd, idsd, block_rows=block_rows, packed=True)
    assert torch.equal(out, out_ref)
    if m <= 256 and block_rows == 0:
        # the decode stages on their own, routes collected from topk_ids
        from litemoe_amd import _lib
        routes = m * k
        act = torch.empty(routes, i, device=DEV, dtype=torch.bfloat16)
        act_ref = experts.gate_up(xd, w1d, None, None, k, topk_ids=idsd.int())
        _lib.call("lm_moe_gate_up_packed", xd.data_ptr(), p1.data_ptr(), None, None, idsd.int().data_ptr(),
                  routes, k, h, i, e, 0, act.data_ptr(), _lib.stream(xd.device))
        assert torch.equal(act, act_ref)
        y = torch.empty(routes, h, device=DEV, dtype=torch.bfloat16)
        _lib.call("lm_moe_down_packed", act.data_ptr(), p2.data_ptr(), None, None, idsd.int().data_ptr(),
                  routes, h, i, e, 0, y.data_ptr(), _lib.stream(xd.device))
        assert torch.equal(y, ref)
    if m <= 16:
        assert rel_l2(got.cpu(), ops.expert_routes(x, ids, w1, w2)) < 1e-2
