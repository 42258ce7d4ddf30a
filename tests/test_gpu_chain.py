"""The chained decode layer: the router's expert-id order, the combine and
residual add fused into the down projection (lm_moe_routes_combine), and the
next RMSNorm formed inside the QKV projection (lm_linear_splitk_rmsnorm).

Bars: bit-exact against the unchained kernels they replace (router ids and
weights in logit order, lm_moe_routes + lm_moe_finish[_add_rmsnorm],
lm_linear_splitk on lm_rmsnorm's output), over repeated calls and graph
replays (the arrival counters reset themselves), and whole decode runs with
the chain on and off.
"""
import pytest
import torch

from litemoe_amd import experts, linear, norm, router
from litemoe_amd.synth import normal_bf16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf(shape, std, seed):
    return normal_bf16(shape, std, seed).to(DEV)


def _sorted_like(weights, ids):
    """Each token's (weight, id) pairs reordered by ascending id."""
    order = ids.long().argsort(dim=1)
    return weights.gather(1, order), ids.gather(1, order)


@pytest.mark.parametrize("m,h,e,k", [(64, 1536, 40, 8), (33, 1024, 32, 8), (16, 512, 100, 6),
                                     (1029, 1536, 40, 8), (7, 256, 8, 2)])
@torch.inference_mode()
def test_router_id_order_is_the_logit_order_sorted(m, h, e, k):
    """renormalize bit 1: the same experts and weights, each token's in
    ascending id (the wave selection for <= 64 experts, the workgroup one
    above, the batched MFMA router from 1024 tokens)."""
    z = bf((m, h), 1.0, m + h)
    wr = bf((e, h), 0.02, e + 1)
    weights, ids = router.route(z, wr, k)
    w_id, ids_id = router.route(z, wr, k, id_order=True)
    exp_w, exp_ids = _sorted_like(weights, ids)
    assert torch.equal(ids_id, exp_ids)
    assert torch.equal(w_id, exp_w)
    assert bool((ids_id[:, 1:] > ids_id[:, :-1]).all())


@torch.inference_mode()
def test_router_splitk_id_order():
    m, h, e, k = 64, 1536, 40, 8
    x0 = bf((m, h), 1.0, 3)
    part = normal_bf16((4, m, h), 0.5, 4).float().to(DEV)
    nw = bf((h,), 1.0, 5)
    wr = bf((e, h), 0.02, 6)
    xa, xb = x0.clone(), x0.clone()
    wa, ia, za = router.add_rmsnorm_route_splitk(xa, part, 0.22, nw, 1e-6, wr, k)
    wb, ib, zb = router.add_rmsnorm_route_splitk(xb, part, 0.22, nw, 1e-6, wr, k, id_order=True)
    assert torch.equal(xa, xb) and torch.equal(za, zb)
    exp_w, exp_ids = _sorted_like(wa, ia)
    assert torch.equal(ib, exp_ids) and torch.equal(wb, exp_w)


def _case(m, h, i, e, k, seed):
    z = bf((m, h), 1.0, seed)
    w1 = bf((e, 2 * i, h), 0.02, seed + 1)
    w2 = bf((e, h, i), 0.02, seed + 2)
    wr = bf((e, h), 0.02, seed + 3)
    weights, ids = router.route(z, wr, k, id_order=True)
    return z, w1, w2, weights, ids


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("m,h,i,e,k", [(64, 1536, 512, 40, 8), (128, 1536, 512, 40, 8), (32, 1024, 512, 32, 8),
                                       (5, 512, 256, 8, 2), (256, 1024, 256, 16, 8), (1, 1536, 512, 40, 8)])
@torch.inference_mode()
def test_routes_combine_equals_routes_and_finish(m, h, i, e, k, packed):
    """Without a residual: out equals lm_fused_experts (gate/up, down, then
    the moe_finish combine). With one: the residual equals
    lm_moe_finish_add_rmsnorm's, and the QKV partials formed from it and the
    sums of squares equal lm_linear_splitk on that kernel's normalised z.
    Twice in a row with new inputs (the counters are left at zero)."""
    r, eps = 0.22, 1e-6
    nw = bf((h,), 1.0, 77)
    wq = bf((2560 if h == 1536 else h, h), 0.02, 78)
    splits = linear.pick_splits(min(m, 128), wq.shape[0], h)
    ws = experts._Workspace()
    for seed in (11, 12):
        z, w1, w2, weights, ids = _case(m, h, i, e, k, seed + m)
        a1, a2 = experts.pack_expert_weights(w1, w2) if packed else (w1, w2)
        ref = experts.fused_experts(z, w1, w2, weights, ids)
        got = experts.moe_routes_combine(z, a1, a2, ids, weights, workspace=ws, packed=packed)
        assert torch.equal(got, ref)
        x0 = bf((m, h), 1.0, seed + 5)
        y = experts.moe_routes(z, w1, w2, ids)
        x_ref = x0.clone()
        z_ref = experts.finish_add_rmsnorm(y, ids, weights, x_ref, r, nw, eps)
        x_new = x0.clone()
        sumsq = experts.moe_routes_combine(z, a1, a2, ids, weights, residual=x_new, alpha=r, workspace=ws,
                                           packed=packed)
        assert torch.equal(x_new, x_ref)
        assert torch.equal(norm.rmsnorm(x_new, nw, eps), z_ref)
        if m <= 128 and splits:
            exp = linear.linear_splitk(z_ref, wq, splits)
            assert torch.equal(linear.linear_splitk_rmsnorm(x_new, sumsq, nw, eps, wq, splits), exp)


@torch.inference_mode()
def test_routes_combine_graph_replays():
    """Recorded into a HIP graph and replayed with new inputs between the
    replays: every replay equals the eager call (the counters reset
    themselves; no memset is recorded)."""
    m, h, i, e, k, r = 64, 1536, 512, 40, 8, 0.22
    z, w1, w2, weights, ids = _case(m, h, i, e, k, 5)
    p1, p2 = experts.pack_expert_weights(w1, w2)
    x = bf((m, h), 1.0, 6)
    sumsq = torch.empty(m, h // 64, device=DEV, dtype=torch.float32)
    ws = experts._Workspace()

    def step():
        experts.moe_routes_combine(z, p1, p2, ids, weights, residual=x, alpha=r, sumsq=sumsq, workspace=ws,
                                   packed=True)

    x_start = x.clone()
    step()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(3):
        zz, _, _, ww, ii = _case(m, h, i, e, k, 20 + rep)
        z.copy_(zz)
        weights.copy_(ww)
        ids.copy_(ii)
        x.copy_(x_start)
        graph.replay()
        torch.cuda.synchronize()
        got_x, got_s = x.clone(), sumsq.clone()
        x.copy_(x_start)
        step()
        torch.cuda.synchronize()
        assert torch.equal(got_x, x) and torch.equal(got_s, sumsq), rep


@pytest.mark.parametrize("name,batch", [("granite-3b", 24), ("granite-1b", 64)])
@torch.inference_mode()
def test_chained_decode_equals_unchained(name, batch):
    """Two layers of the cfg-3 / cfg-2 shape: graph decode with the chain on
    and off gives the same tokens, engine state and KV cache bit for bit."""
    from litemoe_amd import synth
    from litemoe_amd.config import preset
    from litemoe_amd.engine import Request
    from litemoe_amd.ep import ExpertParallel
    from litemoe_amd.experts import HipFusedExperts
    from litemoe_amd.model import Granite
    from litemoe_amd.optimized import OptimizedEngine
    cfg = preset(name, num_hidden_layers=2)
    w = synth.granite_weights(cfg, seed=3, device=DEV, method="torch")
    ep = ExpertParallel(1, 0, 4096, cfg.hidden_size, cfg.num_experts_per_tok, torch.bfloat16, DEV,
                        HipFusedExperts())
    model = Granite(cfg, w, ep, 256)
    model.chain_combine = True
    assert model._combine_chain(batch)
    prompts = synth.prompts(batch, synth.ragged_lengths(batch, 5, 60, 4), cfg.vocab_size, 2)
    requests = [Request(str(j), p, 6) for j, p in enumerate(prompts)]
    runs = []
    for chain in (True, False):
        model.chain_combine = chain
        run = OptimizedEngine(model, requests, ignore_eos=True, capacity=128, mode="graph")
        out, _ = run.generate()
        runs.append((out, {k: v.clone() for k, v in run.state.items()}, run.cache.k.clone(), run.cache.v.clone()))
        del run
    (o1, s1, k1, v1), (o2, s2, k2, v2) = runs
    assert o1 == o2
    assert all(torch.equal(s1[key], s2[key]) for key in s1)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
