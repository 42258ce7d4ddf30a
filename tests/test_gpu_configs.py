"""The benchmark configurations at their own sizes, against the oracle.

* cfg 4: packed ragged prefill of 48 prompts, lengths U{64..2048} (seed 2,
  about 47k tokens), on the Granite-3B shape (two layers) with four hot
  experts taking about half of the routes. The skew is made this way:
  a constant vector c is added to every embedding row and beta * c/|c| to
  the router rows of four hot experts, beta calibrated here so that layer 0
  sends 45-55% of its routes to them. Checked at the full token count:
  router ids bit-exact given the kernel's logits, the route permutation
  bit-exact, sampled route outputs (hot and cold experts) and sampled
  sequences' attention (the longest included) against the oracle, and the
  last-position logits of three whole sequences against the oracle's
  prefill of those sequences (a packed sequence depends on its own tokens
  only).
* cfg 3 at full depth: 32 layers, batch 64, 1024-token prompts; one lean
  decode step's logits on eight rows against the oracle's decode of those
  rows over the GPU-filled KV cache (rounding drift over all 32 layers).
"""
import pytest
import torch

from helpers import rel_l2
from litemoe_amd import experts, packed, router, synth
from litemoe_amd import model as model_module
from litemoe_amd.cache import KVCache
from litemoe_amd.config import preset
from litemoe_amd.ep import ExpertParallel
from litemoe_amd.experts import HipFusedExperts
from litemoe_amd.model import Granite
from litemoe_amd.packed import packed_prefill_logits
from oracle import granite as oracle
from oracle import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
HOT = (3, 17, 26, 38)


def _cpu(w):
    return {k: ([{n: t.cpu() for n, t in layer.items()} for layer in v] if k == "layers" else v.cpu())
            for k, v in w.items()}


class _RouterTap:
    """Records the router inputs and ids of each fused layer call."""

    def __init__(self, monkeypatch):
        self.calls = []
        inner = model_module.route_add_rmsnorm

        def tapped(*args, **kwargs):
            weights, ids, z = inner(*args, **kwargs)
            self.calls.append((z.clone(), ids.clone(), weights.clone()))
            return weights, ids, z

        monkeypatch.setattr(model_module, "route_add_rmsnorm", tapped)


@torch.inference_mode()
def test_cfg4_skewed_packed_prefill_matches_oracle(monkeypatch):
    cfg = preset("granite-3b", num_hidden_layers=2)
    E, k, H = cfg.num_local_experts, cfg.num_experts_per_tok, cfg.hidden_size
    w = synth.granite_weights(cfg, seed=0, device=DEV, method="torch")
    gen = torch.Generator(device=DEV).manual_seed(21)
    c = (torch.randn(H, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    w["embedding"] += c
    c_hat = c.float() / c.float().norm()
    base = [layer["block_sparse_moe.router.layer"].clone() for layer in w["layers"]]
    hot = torch.tensor(HOT, device=DEV)
    lengths = synth.ragged_lengths(48, 64, 2048, 2)
    prompts = synth.prompts(48, lengths, cfg.vocab_size, 1)
    tokens = sum(lengths)
    ep = ExpertParallel(1, 0, tokens, H, k, torch.bfloat16, DEV, HipFusedExperts())
    model = Granite(cfg, w, ep, 4096)
    cache = KVCache(cfg, 48, 2048, DEV, torch.bfloat16)
    tap = _RouterTap(monkeypatch)

    def run(beta):
        for layer, b in zip(w["layers"], base):
            r = b.clone()
            r[hot] = (r[hot].float() + beta * c_hat).to(torch.bfloat16)
            layer["block_sparse_moe.router.layer"].copy_(r)
        tap.calls.clear()
        logits = packed_prefill_logits(model, prompts, cache)[:, 0]
        shares = [float(torch.isin(ids, hot).float().mean()) for _, ids, _ in tap.calls]
        return logits, shares

    lo, hi = 0.0, 4.0
    # Bisection of the layer-0 hot share to 48%: with top-8, four experts
    # chosen by every token is a 50% share, so the target sits just below
    # that saturation.
    for _ in range(14):
        beta = (lo + hi) / 2
        _, shares = run(beta)
        if shares[0] < 0.48:
            lo = beta
        else:
            hi = beta
    logits, shares = run((lo + hi) / 2)
    print(f"cfg4: {tokens} tokens, beta {(lo + hi) / 2:.4f}, hot share per layer {shares}")
    assert 0.45 <= shares[0] <= 0.55
    assert len(tap.calls) == 2

    for layer, (z, ids, weights) in enumerate(tap.calls):
        wl = w["layers"][layer]
        # router: the standalone kernel gives the fused call's ids; ids are the
        # exact top-k of the kernel's own logits
        kernel_logits = torch.empty(tokens, E, device=DEV, dtype=torch.bfloat16)
        w2_, ids2 = router.route(z, wl["block_sparse_moe.router.layer"], k, logits_out=kernel_logits)
        assert torch.equal(ids2, ids) and torch.equal(w2_, weights)
        ew, eids = ops.route(kernel_logits.cpu(), k)
        assert torch.equal(ids.cpu(), eids)
        torch.testing.assert_close(weights.cpu(), ew, rtol=2e-6, atol=1e-7)
        # permutation at the full route count (about 376k routes)
        offsets, order, inverse = experts.moe_align(ids, E)
        eo, eord, einv = ops.permutation(ids.cpu(), E)
        assert offsets.cpu().tolist() == eo.tolist()
        assert torch.equal(order.cpu().long(), eord) and torch.equal(inverse.cpu().long(), einv)
        # expert GEMMs over all routes; sampled routes of hot and cold experts
        y = experts.moe_routes(z, wl["input_linear"], wl["output_linear"], ids)
        flat = ids.reshape(-1).cpu().long()
        g = torch.Generator().manual_seed(layer)
        is_hot = torch.isin(flat, torch.tensor(HOT))
        picks = []
        for mask in (is_hot, ~is_hot):
            cand = mask.nonzero().flatten()
            picks.append(cand[torch.randperm(cand.numel(), generator=g)[:384]])
        sample = torch.cat(picks)
        zc = z.cpu()
        expected = ops.expert_routes(zc[sample // k], flat[sample][:, None], wl["input_linear"].cpu(),
                                     wl["output_linear"].cpu())
        got = y.cpu()[sample]
        assert rel_l2(got[:384], expected[:384]) < 1e-2  # hot
        assert rel_l2(got[384:], expected[384:]) < 1e-2  # cold
        per_route = (got.float() - expected.float()).norm(dim=1) / expected.float().norm(dim=1).clamp_min(1e-6)
        assert float(per_route.max()) < 5e-2

    # attention over the whole packed batch; three sequences against the oracle
    hq, hkv = cfg.num_attention_heads, cfg.num_key_value_heads
    q = torch.randn(tokens, hq, 64, device=DEV, generator=gen).to(torch.bfloat16)
    kk = torch.randn(tokens, hkv, 64, device=DEV, generator=gen).to(torch.bfloat16)
    vv = torch.randn(tokens, hkv, 64, device=DEV, generator=gen).to(torch.bfloat16)
    ends = torch.tensor(lengths, dtype=torch.int32).cumsum(0, dtype=torch.int32)
    cu = torch.cat((ends.new_zeros(1), ends))
    out = packed.varlen_attention(q, kk, vv, cu.to(DEV), max(lengths), cfg.attention_multiplier).cpu()
    chosen = sorted({lengths.index(max(lengths)), lengths.index(min(lengths)), 24})
    for s in chosen:
        a, b = int(cu[s]), int(cu[s + 1])
        exp = ops.varlen_attention(q[a:b].cpu(), kk[a:b].cpu(), vv[a:b].cpu(), torch.tensor([0, b - a]),
                                   cfg.attention_multiplier)
        torch.testing.assert_close(out[a:b], exp, atol=.016, rtol=.016)  # reference test_packed_prefill.py:40

    # last-position logits of whole sequences against the oracle's prefill
    ref = oracle.Granite(cfg, _cpu(w), 2048, fused=True)
    rcache = oracle.Cache(cfg, 1, 2048, torch.bfloat16)
    got = logits.cpu()
    for s in chosen:
        exp = ref.prefill(prompts[s], rcache, 0, last_only=True)[0]
        assert rel_l2(got[s], exp) < 2e-2, (s, lengths[s])
        assert int(got[s].float().argmax()) == int(exp.float().argmax()) or \
            float(exp.float().max() - exp.float()[int(got[s].float().argmax())]) < 0.05


@torch.inference_mode()
def test_cfg3_full_depth_decode_step_matches_oracle():
    cfg = preset("granite-3b")
    batch, prompt_len, cap = 64, 1024, 2048
    w = synth.granite_weights(cfg, seed=0, device=DEV, method="torch")
    ep = ExpertParallel(1, 0, batch * prompt_len, cfg.hidden_size, cfg.num_experts_per_tok, torch.bfloat16,
                        DEV, HipFusedExperts())
    model = Granite(cfg, w, ep, cap)
    prompts = synth.prompts(batch, prompt_len, cfg.vocab_size, 1)
    cache = KVCache(cfg, batch, cap, DEV, torch.bfloat16)
    first = packed_prefill_logits(model, prompts, cache)[:, 0].argmax(-1)
    lengths = torch.full((batch,), prompt_len, device=DEV)
    valid = torch.ones(batch, dtype=torch.bool, device=DEV)
    model.decode_lean = model.ep.decode_lean = True
    got = model.forward(first[:, None], lengths[:, None], valid[:, None], cache)[:, 0].cpu()
    rows = torch.tensor([0, 5, 13, 22, 31, 40, 51, 63])
    sub = oracle.Granite(cfg, _cpu(w), cap, fused=True)
    rcache = oracle.Cache(cfg, rows.numel(), cap, torch.bfloat16)
    # the cache as the GPU left it before this step: positions 0..1023 (the
    # step has since written position 1024, which the oracle writes itself)
    rcache.k[:, :, :, :prompt_len] = cache.k[:, rows.to(DEV), :, :prompt_len].cpu()
    rcache.v[:, :, :, :prompt_len] = cache.v[:, rows.to(DEV), :, :prompt_len].cpu()
    exp = sub.decode(first.cpu()[rows], lengths.cpu()[rows], torch.ones(rows.numel(), dtype=torch.bool), rcache)
    err = rel_l2(got[rows], exp)
    agree = int((got[rows].float().argmax(-1) == exp.float().argmax(-1)).sum())
    print(f"cfg3 full depth: logits rel-L2 {err:.3e}, argmax agreement {agree}/{rows.numel()}")
    assert err < 2e-2
    assert agree >= rows.numel() - 1
    # the KV the step wrote at position 1024 for these rows, all 32 layers
    assert rel_l2(cache.k[:, rows.to(DEV), :, prompt_len].cpu(), rcache.k[:, :, :, prompt_len]) < 2e-2
