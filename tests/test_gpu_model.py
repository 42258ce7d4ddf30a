"""Model- and engine-level parity of the gfx950 path.

The product ``Granite`` (all hot ops on the HIP kernels) against the CPU
oracle with the production rounding (``fused=True``) on a 64-dim-head Granite
geometry; logits within rel-L2 2e-2, greedy argmax agreement reported; the
engine's eager, graph and graph-async modes give identical outputs.
"""
import pytest
import torch

from helpers import config_from_hf, hf_weights, make_hf, rel_l2
from litemoe_amd.cache import KVCache
from litemoe_amd.engine import Engine, Request
from litemoe_amd.ep import ExpertParallel
from litemoe_amd.experts import HipFusedExperts
from litemoe_amd.model import Granite
from litemoe_amd.optimized import OptimizedEngine, optimized_policy
from litemoe_amd.packed import packed_prefill_logits
from oracle import granite as oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
GEOMETRY = dict(vocab_size=97, hidden_size=256, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
                num_key_value_heads=2, num_local_experts=8, num_experts_per_tok=2, max_position_embeddings=256)


def build(seed=3, capacity=64, **overrides):
    hf = make_hf(seed=seed, **{**GEOMETRY, **overrides})
    cfg = config_from_hf(hf.config)
    w_cpu = hf_weights(hf, torch.bfloat16)
    w_gpu = hf_weights(hf, torch.bfloat16, DEV)
    ep = ExpertParallel(1, 0, 4096, cfg.hidden_size, cfg.num_experts_per_tok, torch.bfloat16, DEV,
                        HipFusedExperts())
    return hf, cfg, Granite(cfg, w_gpu, ep, capacity), oracle.Granite(cfg, w_cpu, capacity, fused=True)


@pytest.mark.parametrize("lean", [False, True])
@torch.inference_mode()
def test_prefill_and_decode_logits_match_oracle(lean):
    hf, cfg, model, ref = build()
    prompts = [[5, 17, 3, 44, 8, 90], [2], [7, 7, 7, 1, 60, 33, 21, 9, 4, 80, 11]]
    cap = 64
    cache = KVCache(cfg, len(prompts), cap, DEV, torch.bfloat16)
    rcache = oracle.Cache(cfg, len(prompts), cap, torch.bfloat16)
    logits = packed_prefill_logits(model, prompts, cache)[:, 0].cpu()
    expected = torch.stack([ref.prefill(p, rcache, j)[-1] for j, p in enumerate(prompts)])
    assert rel_l2(logits, expected) < 2e-2
    assert torch.equal(logits.argmax(-1), expected.argmax(-1))
    for layer in range(cfg.num_hidden_layers):
        for j, p in enumerate(prompts):
            assert rel_l2(cache.k[layer, j, :, :len(p)].cpu(), rcache.k[layer, j, :, :len(p)]) < 2e-2
    assert cache.k[:, 1, :, 1:].count_nonzero() == 0  # nothing past a prompt
    tokens = expected.argmax(-1)
    lengths = torch.tensor([len(p) for p in prompts])
    model.decode_lean = model.ep.decode_lean = lean
    agree, steps = 0, 0
    for step in range(5):
        valid = torch.tensor([True, step < 2, True])
        positions = torch.where(valid, lengths, 0)
        got = model.forward(tokens[:, None].to(DEV), positions[:, None].to(DEV), valid[:, None].to(DEV),
                            cache)[:, 0].cpu()
        exp = ref.decode(tokens, positions, valid, rcache)
        assert rel_l2(got[valid], exp[valid]) < 2e-2
        agree += int((got.argmax(-1) == exp.argmax(-1))[valid].sum())
        steps += int(valid.sum())
        tokens = torch.where(valid, exp.argmax(-1), tokens)
        lengths += valid
    assert agree >= steps - 1


@pytest.mark.parametrize("name", ["granite-1b", "granite-3b"])
@torch.inference_mode()
def test_benchmark_shapes_prefill_and_decode_match_oracle(name):
    """cfg 2 / cfg 3 per-layer shapes (hidden 1024 / 1536, 16/8 and 24/8
    heads, 32 / 40 experts top-8, intermediate 512, vocab 49155) with two
    layers of random bf16 weights: packed prefill of four ragged prompts,
    then lean decode steps (split-K projections, fused attention, fused
    router, scan-path experts, greedy epilogue shapes) against the oracle's
    production rounding. Logits within rel-L2 2e-2 per step, greedy argmax
    agreement."""
    from litemoe_amd import synth
    from litemoe_amd.config import preset
    cfg = preset(name, num_hidden_layers=2)
    w_gpu = synth.granite_weights(cfg, seed=4, device=DEV, method="torch")
    w_cpu = {k: ([{n: t.cpu() for n, t in layer.items()} for layer in v] if k == "layers" else v.cpu())
             for k, v in w_gpu.items()}
    ep = ExpertParallel(1, 0, 4096, cfg.hidden_size, cfg.num_experts_per_tok, torch.bfloat16, DEV,
                        HipFusedExperts())
    cap = 64
    model, ref = Granite(cfg, w_gpu, ep, cap), oracle.Granite(cfg, w_cpu, cap, fused=True)
    prompts = synth.prompts(4, [23, 9, 40, 17], cfg.vocab_size, 6)
    cache = KVCache(cfg, len(prompts), cap, DEV, torch.bfloat16)
    rcache = oracle.Cache(cfg, len(prompts), cap, torch.bfloat16)
    logits = packed_prefill_logits(model, prompts, cache)[:, 0].cpu()
    expected = torch.cat([ref.prefill(p, rcache, j, last_only=True) for j, p in enumerate(prompts)])
    assert rel_l2(logits, expected) < 2e-2
    assert int((logits.argmax(-1) == expected.argmax(-1)).sum()) >= 3
    tokens = expected.argmax(-1)
    lengths = torch.tensor([len(p) for p in prompts])
    model.decode_lean = model.ep.decode_lean = True
    agree, steps = 0, 0
    for step in range(4):
        valid = torch.ones(len(prompts), dtype=torch.bool)
        got = model.forward(tokens[:, None].to(DEV), lengths[:, None].to(DEV), valid[:, None].to(DEV),
                            cache)[:, 0].cpu()
        exp = ref.decode(tokens, lengths, valid, rcache)
        assert rel_l2(got, exp) < 2e-2, step
        agree += int((got.argmax(-1) == exp.argmax(-1)).sum())
        steps += len(prompts)
        tokens = exp.argmax(-1)
        lengths += 1
    assert agree >= steps - 1


@torch.inference_mode()
def test_decode_above_128_rows_matches_oracle():
    """A decode batch of 136 rows on the cfg 3 layer shape (two layers): the
    projections run on lm_linear (QKV with the RoPE/KV epilogue), attention
    on lm_flash_decode, the experts on the grouped path and the head on
    lm_linear; packed prefill first, then decode steps against the oracle's
    production rounding (logits within rel-L2 2e-2, greedy argmax agreement),
    and a graph-mode greedy generate that emits the oracle's first token."""
    from litemoe_amd import synth
    from litemoe_amd.config import preset
    cfg = preset("granite-3b", num_hidden_layers=2)
    w_gpu = synth.granite_weights(cfg, seed=5, device=DEV, method="torch")
    w_cpu = {k: ([{n: t.cpu() for n, t in layer.items()} for layer in v] if k == "layers" else v.cpu())
             for k, v in w_gpu.items()}
    ep = ExpertParallel(1, 0, 4096, cfg.hidden_size, cfg.num_experts_per_tok, torch.bfloat16, DEV,
                        HipFusedExperts())
    cap, batch = 32, 136
    model, ref = Granite(cfg, w_gpu, ep, cap), oracle.Granite(cfg, w_cpu, cap, fused=True)
    assert model.decode_splits(batch) is None  # above the split-K kernels' 128 rows
    prompts = synth.prompts(batch, synth.ragged_lengths(batch, 3, 12, 7), cfg.vocab_size, 8)
    cache = KVCache(cfg, batch, cap, DEV, torch.bfloat16)
    rcache = oracle.Cache(cfg, batch, cap, torch.bfloat16)
    logits = packed_prefill_logits(model, prompts, cache)[:, 0].cpu()
    expected = torch.cat([ref.prefill(p, rcache, j, last_only=True) for j, p in enumerate(prompts)])
    assert rel_l2(logits, expected) < 2e-2
    tokens = expected.argmax(-1)
    lengths = torch.tensor([len(p) for p in prompts])
    agree, steps = 0, 0
    for step in range(3):
        valid = torch.ones(batch, dtype=torch.bool)
        valid[::17] = step < 1  # some rows stop after the first step
        positions = torch.where(valid, lengths, 0)
        got = model.forward(tokens[:, None].to(DEV), positions[:, None].to(DEV), valid[:, None].to(DEV),
                            cache)[:, 0].cpu()
        exp = ref.decode(tokens, positions, valid, rcache)
        assert rel_l2(got[valid], exp[valid]) < 2e-2, step
        agree += int((got.argmax(-1) == exp.argmax(-1))[valid].sum())
        steps += int(valid.sum())
        tokens = torch.where(valid, exp.argmax(-1), tokens)
        lengths += valid
    assert agree >= steps - 2
    requests = [Request(str(j), p, 3) for j, p in enumerate(prompts)]
    out, _ = OptimizedEngine(model, requests, ignore_eos=True, capacity=cap, mode="graph").generate()
    first = expected.argmax(-1)
    assert sum(out[str(j)][0] == int(first[j]) for j in range(batch)) >= batch - 2


@torch.inference_mode()
def test_engine_modes_identical_and_close_to_oracle_greedy():
    """Reference test_cuda_execution.py:102-133: graph and graph-async equal
    eager, repeated generate() calls agree, EOS/poll inside the graph."""
    hf, cfg, model, ref = build(seed=5)
    requests = [Request("a", [3, 8, 2], 7), Request("b", [4], 2), Request("c", [9, 2], 1)]
    eager, _ = OptimizedEngine(model, requests, ignore_eos=True, capacity=16).generate()
    for mode in ("graph", "graph-async"):
        engine = OptimizedEngine(model, requests, mode=mode, ignore_eos=True, capacity=16)
        for _ in range(3):
            actual, metrics = engine.generate()
            assert actual == eager
            assert metrics["output_tokens"] == 10 and metrics["decode_tokens"] == 7
            assert engine.state["length"].tolist() == [9, 2, 2]
    outputs, _ = oracle.generate(ref, [r.prompt for r in requests], [r.budget for r in requests], 16)
    same = sum(a == b for r, o in zip(requests, outputs) for a, b in zip(eager[r.request_id], o))
    assert same >= 8  # greedy agreement on 10 tokens (bf16 ties may flip late tokens)
    model.cfg.eos_token_id = eager["a"][0]
    expected, _ = OptimizedEngine(model, requests, poll=4, capacity=16).generate()
    assert expected["a"] == [eager["a"][0]]
    for mode in ("graph", "graph-async"):
        engine = OptimizedEngine(model, requests, mode=mode, poll=4, capacity=16)
        actual, _ = engine.generate()
        assert actual == expected
        assert not engine.state["active"].any()


@torch.inference_mode()
def test_lean_decode_never_writes_stopped_rows():
    """Reference test_lean_decode.py:32-48: rows that stop keep their KV."""
    hf, cfg, model, ref = build(seed=9)
    requests = [Request("stops", [2, 3, 5], 2), Request("long", [7, 11], 8), Request("mid", [13], 4),
                Request("one", [17], 1)]
    run = OptimizedEngine(model, requests, capacity=16, ignore_eos=True)
    outputs, _ = run.generate()
    assert {k: len(v) for k, v in outputs.items()} == {"stops": 2, "long": 8, "mid": 4, "one": 1}
    assert not run.cache.k[:, 3, :, 1:].count_nonzero() and not run.cache.v[:, 3, :, 1:].count_nonzero()
    assert not run.cache.k[:, 0, :, 4:].count_nonzero() and not run.cache.v[:, 0, :, 4:].count_nonzero()
    with optimized_policy(run):
        assert model.decode_lean and model.ep.decode_lean
    assert not model.decode_lean


@torch.inference_mode()
def test_granite_1b_shape_layer_graph_replay_is_deterministic():
    """cfg-2 geometry (H 1024, 16/8 heads, 32 experts top-8, I 512) with two
    layers: graph replays equal eager bit for bit (no atomics anywhere)."""
    from litemoe_amd import synth
    from litemoe_amd.config import preset
    cfg = preset("granite-1b", num_hidden_layers=2, vocab_size=1000)
    w = synth.granite_weights(cfg, seed=1, device=DEV, method="torch")
    ep = ExpertParallel(1, 0, 4096, cfg.hidden_size, 8, torch.bfloat16, DEV, HipFusedExperts())
    model = Granite(cfg, w, ep, 1024)
    prompts = synth.prompts(32, 100, cfg.vocab_size, 1)
    run = OptimizedEngine(model, [Request(str(i), p, 6) for i, p in enumerate(prompts)], ignore_eos=True,
                          capacity=128)
    eager, _ = run.generate()
    run_g = OptimizedEngine(model, [Request(str(i), p, 6) for i, p in enumerate(prompts)], ignore_eos=True,
                            capacity=128, mode="graph")
    for _ in range(2):
        assert run_g.generate()[0] == eager


def _cache_difference(part, mode, got, exp):
    """Where two KV caches [layers, rows, kv heads, positions, 64] differ."""
    ne = got.view(torch.int16) != exp.view(torch.int16)
    layers = ne.flatten(1).any(1).nonzero().flatten().tolist()
    positions = ne.any(4).any(2).any(1).any(0).nonzero().flatten().tolist()
    rows = ne.any(4).any(3).any(2).any(0).nonzero().flatten().tolist()
    return (f"{mode}: cache.{part} differs in {int(ne.sum())} elements; layers {layers[:8]}, "
            f"rows {rows[:8]} ({len(rows)}), positions {positions[:4]}..{positions[-4:]}")


@pytest.mark.parametrize("name,batch,lengths,capacity", [
    ("granite-3b", 64, 1024, 2048),                   # cfg 3, the headline configuration
    ("granite-1b", 32, 512, 1024),                    # cfg 2
    ("granite-3b", 128, (1024, 4032, 3), 4096)])      # cfg 5: ragged, rows dispatched longest first
@torch.inference_mode()
def test_full_size_graph_replay_equals_eager(name, batch, lengths, capacity):
    """The benchmark configurations at full size (all layers, vocab 49155):
    the hipGraph decode replays give the eager tokens, state and KV cache
    bit for bit, on two generate() calls; every emitted token is in the
    vocabulary."""
    from litemoe_amd import synth
    from litemoe_amd.config import preset
    cfg = preset(name)
    if isinstance(lengths, tuple):
        lengths = synth.ragged_lengths(batch, *lengths)
    w = synth.granite_weights(cfg, seed=0, device=DEV, method="torch")
    total = lengths * batch if isinstance(lengths, int) else sum(lengths)
    ep = ExpertParallel(1, 0, total, cfg.hidden_size, cfg.num_experts_per_tok, torch.bfloat16, DEV,
                        HipFusedExperts())
    model = Granite(cfg, w, ep, capacity)
    prompts = synth.prompts(batch, lengths, cfg.vocab_size, 1)
    requests = [Request(str(i), p, 5) for i, p in enumerate(prompts)]
    eager_run = OptimizedEngine(model, requests, ignore_eos=True, capacity=capacity)
    eager, _ = eager_run.generate()
    assert all(len(t) == 5 and all(0 <= x < cfg.vocab_size for x in t) for t in eager.values())
    for mode in ("graph", "graph-async"):  # graph-async: the epilogue writes the pinned emit ring
        graph_run = OptimizedEngine(model, requests, ignore_eos=True, capacity=capacity, mode=mode)
        for _ in range(2):
            actual, metrics = graph_run.generate()
            assert actual == eager
            assert metrics["output_tokens"] == batch * 5
            for k in eager_run.state:
                assert torch.equal(graph_run.state[k], eager_run.state[k]), k
            # both caches are compared before anything is asserted, so a
            # mismatch reports K and V together
            differences = [_cache_difference(part, mode, getattr(graph_run.cache, part),
                                             getattr(eager_run.cache, part))
                           for part in ("k", "v")
                           if not torch.equal(getattr(graph_run.cache, part), getattr(eager_run.cache, part))]
            assert not differences, "; ".join(differences)
        del graph_run
    del eager_run, model, w
    torch.cuda.empty_cache()



@torch.inference_mode()
def test_padded_prefill_matches_oracle_and_zeroes_padding():
    """The reference's right-padded prefill (litemoe/batch.py:14-21 ->
    model.forward(slot=slice, last=lengths-1), cache.py:21-33): last-position
    logits against the oracle's per-request prefill (rel-L2 2e-2, argmax
    equal), KV of every prompt position against the oracle's cache, zeros in
    the padding positions of each row, and untouched rows outside the slice."""
    from litemoe_amd import batch
    hf, cfg, model, ref = build(seed=6)
    prompts = [[5, 17, 3, 44, 8, 90], [2], [7, 7, 7, 1, 60, 33, 21, 9, 4, 80, 11], [31, 8]]
    cap = 32
    cache = KVCache(cfg, len(prompts) + 1, cap, DEV, torch.bfloat16)
    cache.k.fill_(1.0)  # stale contents: padding positions must be cleared
    cache.v.fill_(1.0)
    rcache = oracle.Cache(cfg, len(prompts) + 1, cap, torch.bfloat16)
    logits = batch.prefill_logits(model, prompts, cache, slot_start=1)[:, 0].cpu()
    expected = torch.stack([ref.prefill(p, rcache, j + 1)[-1] for j, p in enumerate(prompts)])
    assert rel_l2(logits, expected) < 2e-2
    assert torch.equal(logits.argmax(-1), expected.argmax(-1))
    width = max(map(len, prompts))
    for j, p in enumerate(prompts):
        row = j + 1
        for part, rpart in ((cache.k, rcache.k), (cache.v, rcache.v)):
            assert rel_l2(part[:, row, :, :len(p)].cpu(), rpart[:, row, :, :len(p)]) < 2e-2
            assert part[:, row, :, len(p):width].count_nonzero() == 0
            assert bool((part[:, row, :, width:] == 1).all())  # past the batch width: untouched
    assert bool((cache.k[:, 0] == 1).all()) and bool((cache.v[:, 0] == 1).all())  # row outside the slice


@torch.inference_mode()
def test_padded_forward_int_slot_all_positions_and_padding_logits():
    """forward(slot=int) as the reference's plain engine calls it, and
    last=None on a padded row: valid positions match the packed prefill of
    the same prompt; a padding position's logits are those of
    norm(embedding * multiplier), its residual stream untouched by the
    layers (attention masked, zero expert rows in the reference)."""
    from litemoe_amd.norm import rmsnorm
    hf, cfg, model, ref = build(seed=7)
    prompt = [4, 9, 22, 61, 3]
    width = 8
    cache = KVCache(cfg, 2, 16, DEV, torch.bfloat16)
    tokens = torch.tensor([prompt + [0] * (width - len(prompt))], device=DEV)
    positions = torch.arange(width, device=DEV)[None]
    valid = positions < len(prompt)
    all_logits = model.forward(tokens, positions, valid, cache, slot=1)[0].cpu()
    assert all_logits.shape == (width, cfg.vocab_size)
    one = model.forward(tokens, positions, valid, cache, slot=1, last=len(prompt) - 1)
    assert one.shape == (1, 1, cfg.vocab_size)
    packed_cache = KVCache(cfg, 2, 16, DEV, torch.bfloat16)
    exp = packed_prefill_logits(model, [prompt], packed_cache, 1)[:, 0].cpu()
    assert torch.equal(one[:, 0].cpu(), exp)
    assert torch.equal(all_logits[len(prompt) - 1], exp[0])
    assert torch.equal(cache.k, packed_cache.k) and torch.equal(cache.v, packed_cache.v)
    x = model.w["embedding"][0] * cfg.embedding_multiplier
    pad = (rmsnorm(x[None], model.w["norm"], cfg.rms_norm_eps).float() @ model.w["head"].float().T
           / cfg.logits_scaling).cpu()
    assert rel_l2(all_logits[len(prompt):], pad.expand(width - len(prompt), -1)) < 1e-2
    with pytest.raises(ValueError, match="right-padded"):
        model.forward(tokens, positions, ~valid, cache, slot=1)
    with pytest.raises(ValueError, match="slots"):
        model.forward(tokens, positions, valid, cache, slot=slice(0, 2))


@torch.inference_mode()
def test_plain_and_batched_engines_generate_like_the_optimized_engine():
    """The reference's plain Engine (one forward per request, slot=j,
    litemoe/engine.py:128-148) and BatchPrefillEngine (one padded call) run
    on this model; their greedy tokens agree with the optimized engine's
    (packed prefill) and with the oracle's greedy decode."""
    from litemoe_amd.batch import BatchPrefillEngine
    hf, cfg, model, ref = build(seed=8)
    requests = [Request("a", [3, 8, 2, 40], 6), Request("b", [4], 3), Request("c", [9, 2, 17], 5)]
    optimized, _ = OptimizedEngine(model, requests, ignore_eos=True, capacity=16).generate()
    outputs, _ = oracle.generate(ref, [r.prompt for r in requests], [r.budget for r in requests], 16)
    for cls in (Engine, BatchPrefillEngine):
        got, metrics = cls(model, requests, ignore_eos=True, capacity=16).generate()
        assert metrics["output_tokens"] == 14
        same = sum(a == b for r in requests for a, b in zip(got[r.request_id], optimized[r.request_id]))
        assert same >= 12, (cls.__name__, got, optimized)
        first = [got[r.request_id][0] for r in requests]
        assert sum(a == o[0] for a, o in zip(first, outputs)) >= 2  # bf16 near-ties may flip one


@torch.inference_mode()
def test_model_without_packed_copies_generates_the_same_tokens():
    """pack_weights=False: no fragment-order copies of the experts or the
    head; decode reads the checkpoint layout (the same scan kernels) and the
    head goes through lm_linear and the greedy epilogue. Greedy tokens agree
    with the packed model (the head's logits may differ by one bf16 ulp)."""
    hf, cfg, model, ref = build(seed=11)
    plain = Granite(cfg, model.w, model.ep, 64, pack_weights=False)
    requests = [Request(str(i), p, 6) for i, p in enumerate([[3, 8, 2, 40], [4], [9, 2, 17], [60, 1]])]
    packed_out, _ = OptimizedEngine(model, requests, ignore_eos=True, capacity=16, mode="graph").generate()
    assert plain.packed_head is None
    plain_out, _ = OptimizedEngine(plain, requests, ignore_eos=True, capacity=16, mode="graph").generate()
    same = sum(a == b for r in requests for a, b in zip(packed_out[r.request_id], plain_out[r.request_id]))
    assert same >= 22
