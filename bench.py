#!/usr/bin/env python3
"""Decode throughput of the Granite-3B-shaped MoE on one MI355X.

Workload: Granite-3.1-3B-a800m shape (32 layers, hidden
1536, 24/8 heads, 40 experts top-8, intermediate 512, vocab 49155), random
bf16 weights, batch 64, random prompts of 1024 tokens, 256 new tokens, greedy,
each decode step replayed as one hipGraph.

A "step" is one decode step of the whole batch (64 tokens). After prefill,
W untimed steps run and the state is restored; then exactly K steps are timed
between device synchronisations (K = 255 covers the whole 256-token
generation, context 1024 -> 1279). ``value`` = 64 * K / elapsed.

Also reported on the same JSON line:
  roofline      the dominant kernel (expert gate/up GEMM on the fragment-order
                weights), timed with HIP events over all 32 layers' weights
                (no cache reuse across launches; the 32 launches recorded
                into a HIP graph and replayed), against 8 TB/s;
  fused_moe     the whole per-layer MoE as the decode step runs it (expert
                routes, then combine + residual add + next norm), timed the
                same way;
  cpu_baseline  the CPU oracle (LiteMoE's torch CPU decode path restated) on a
                bounded sample of the same decode step, extrapolated;
  engine_decode_tps  the reference's own metric from Engine.generate()
                (decode_tokens / decode_s with the async output ring).

Two other benchmark configurations print their own JSON line (not the
driver's decode line):
  --prefill       cfg 4: packed prefill of 48 prompts, lengths U{64..2048}
                  (seed 2), on the 3B shape: prefill tok/s, and the MFMA
                  utilisation of the prefill MoE (uniform routes and 50% of
                  routes on 4 hot experts) and of the prefill attention at
                  the same token counts;
  --flash-decode  cfg 5: decode attention over B=128 rows with contexts
                  U{1024..4096} (seed 3), capacity 4096, KV filled N(0,1):
                  GB/s of the KV stream against 8 TB/s;
  --long-decode   cfg 5: the whole hipGraph decode step at B=128 with
                  prompts U{1024..4032} (seed 3), capacity 4096: step tok/s.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "decode tok/s, Granite-3B-shape bf16 bs=64; fused-MoE HBM GB/s % of peak"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=255)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--prompt", type=int, default=1024)
    ap.add_argument("--new-tokens", type=int, default=256)
    ap.add_argument("--model", default="granite-3b")
    ap.add_argument("--roofline-reps", type=int, default=10)
    ap.add_argument("--cpu-layers", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-engine", action="store_true")
    ap.add_argument("--chained", action="store_true",
                    help="decode layers with the combine fused into the down projection and the next norm "
                         "into the QKV projection (Granite.chain_combine)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="skip decode timing: run only the MoE kernel timing (for counter collection)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only copy a 256 MiB device buffer 3 times (FETCH/WRITE counter calibration)")
    ap.add_argument("--read-probe", action="store_true",
                    help="only sum 2048 contiguous 128 KiB rows of a 256 MiB buffer 3 times (a second "
                         "FETCH_SIZE calibration, in the decode attention's per-row access pattern)")
    ap.add_argument("--prefill", action="store_true", help="cfg 4 packed prefill (own JSON line)")
    ap.add_argument("--flash-decode", action="store_true", help="cfg 5 decode attention (own JSON line)")
    ap.add_argument("--long-decode", action="store_true", help="cfg 5 decode step tok/s (own JSON line)")
    return ap.parse_args()


def measured_traffic(name):
    """HBM bytes per launch of a kernel from its committed counter summary
    (FETCH_SIZE + WRITE_SIZE, calibrated on a plain copy), or None."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch="):
                return int(line.split("=", 1)[1])
    except OSError:
        pass
    return None


def moe_roofline(model, cfg, batch, reps):
    """Time the gate/up kernel and the decode step's whole MoE per layer
    (expert routes, then combine + residual add + next norm, as
    ``Granite._fused_layers`` runs them) with HIP events, rotating over every
    layer's weights. Each loop over the 32 layers is recorded into a HIP
    graph and replayed, so the figures are GPU time, not Python time."""
    import torch

    from litemoe_amd import _lib, experts, router
    from litemoe_amd.execution import no_collection_while_recording
    dev = model.w["embedding"].device
    H, I, E, k = cfg.hidden_size, cfg.intermediate_size, cfg.num_local_experts, cfg.num_experts_per_tok
    gen = torch.Generator(device=dev).manual_seed(7)
    z = torch.randn(batch, H, device=dev, generator=gen).to(torch.bfloat16)
    x = torch.randn(batch, H, device=dev, generator=gen).to(torch.bfloat16)
    z_out = torch.empty_like(z)
    # the step's MoE: chained (ids in expert order, the combine and residual
    # add in the down launch) or gate/up, down and combine+add+norm
    chained = model._combine_chain(batch)
    per_layer = []
    for w in model.w["layers"]:
        weights, ids = router.route(z, w["block_sparse_moe.router.layer"], k, id_order=chained)
        act = torch.empty(batch * k, I, device=dev, dtype=torch.bfloat16)
        y = torch.empty(batch * k, H, device=dev, dtype=torch.bfloat16)
        active = int(torch.unique(ids).numel())
        per_layer.append((w, weights, ids, act, y, active))
    # the weights the decode step reads: the fragment layout when the model packed them
    packed = "input_linear_packed" in model.w["layers"][0]
    w13_key, w2_key = ("input_linear_packed", "output_linear_packed") if packed else ("input_linear",
                                                                                      "output_linear")
    backend = model.ep.backend  # its workspace, as the model's fused tail uses it
    r, eps = cfg.residual_multiplier, cfg.rms_norm_eps
    x0 = x.clone()

    def gate_up_all():  # the decode path: each expert's workgroups collect its routes
        stream = _lib.stream(dev)
        for w, weights, ids, act, y, _ in per_layer:
            _lib.call("lm_moe_gate_up_packed" if packed else "lm_moe_gate_up", z.data_ptr(),
                      w[w13_key].data_ptr(), None, None, ids.data_ptr(), batch * k, k, H, I, E, 0,
                      act.data_ptr(), stream)

    sumsq = torch.empty(batch, H // 64, device=dev, dtype=torch.float32)

    def moe_all():
        for w, weights, ids, act, y, _ in per_layer:
            if chained:
                backend.routes_combine(z, w[w13_key], w[w2_key], ids, weights, residual=x, alpha=r, sumsq=sumsq,
                                       packed=packed)
            else:
                experts.moe_routes(z, w[w13_key], w[w2_key], ids, workspace=backend.workspace, y=y,
                                   packed=packed)
                experts.finish_add_rmsnorm(y, ids, weights, x, r, w["post_attention_layernorm"], eps, z_out)

    result = {}
    for name, fn in (("gate_up", gate_up_all), ("fused", moe_all)):
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()  # workspaces allocated outside the recording
            side.synchronize()
            with no_collection_while_recording(), torch.cuda.graph(graph, stream=side):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        graph.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        result[name] = start.elapsed_time(end) * 1e3 / (reps * len(per_layer))  # us per launch / layer
    x.copy_(x0)
    active = sum(p[-1] for p in per_layer) / len(per_layer)
    # Algorithmic bytes (weights of active experts + activations in/out).
    gate_up_bytes = active * 2 * I * H * 2 + batch * H * 2 + batch * k * I * 2
    fused_bytes = active * 3 * I * H * 2 + 2 * batch * H * 2 + batch * k * 8
    return dict(gate_up_us=result["gate_up"], fused_us=result["fused"], active=active,
                gate_up_bytes=gate_up_bytes, fused_bytes=fused_bytes, chained=chained)


def decode_attention_rate(engine, cfg, reps):
    """The decode attention over the engine's own KV cache after the timed
    steps (every layer once per replay of a HIP graph, so nothing is cached
    between layers): ``lm_flash_decode`` with the step's split plan. Bytes:
    the K and V of every used position, plus q and the output."""
    import torch

    from litemoe_amd.execution import no_collection_while_recording
    dev = engine.cache.k.device
    batch, hq, hkv, d = engine.batch, cfg.num_attention_heads, cfg.num_key_value_heads, 64
    used = engine.state["length"].to(torch.int32)
    gen = torch.Generator(device=dev).manual_seed(9)
    q = torch.randn(batch, hq, 1, d, device=dev, generator=gen).to(torch.bfloat16)
    zeros = torch.zeros(batch, dtype=torch.int64, device=dev)
    active = torch.ones(batch, dtype=torch.bool, device=dev)
    flash, cache = engine.flash_attention, engine.cache

    def all_layers():
        for layer in range(cfg.num_hidden_layers):
            flash(q, cache.k[layer], cache.v[layer], zeros, active, cfg.attention_multiplier, used=used)

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        all_layers()
        side.synchronize()
        with no_collection_while_recording(), torch.cuda.graph(graph, stream=side):
            all_layers()
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / (reps * cfg.num_hidden_layers)
    keys = int(used.sum())
    nbytes = keys * hkv * d * 2 * 2 + 2 * batch * hq * d * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"kernel": "decode_kernel (lm_flash_decode)", "achieved": round(gbs, 1), "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "us_per_layer": round(us, 2), "bytes_per_layer": nbytes,
            "mean_context": round(keys / batch, 1)}


BF16_PEAK_TFLOPS = 2500.0


def hip_time(fn, reps):
    """Average milliseconds per call of ``fn`` on the current stream."""
    import torch
    fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def skewed_prefill(model, engine, cfg, dev):
    """cfg 4's skewed router on the model in place, then restored: a constant
    vector c (seed 21) added to every embedding row and beta * c/|c| to the
    router rows of four hot experts, beta bisected so that layer 0 sends 48%
    of its routes to them (with top-8, four experts chosen by every token is
    a 50% share); the prefill timed with that router."""
    import torch

    from litemoe_amd import model as model_module
    hot_ids = (3, 17, 26, 38)
    hot = torch.tensor(hot_ids, device=dev)
    gen = torch.Generator(device=dev).manual_seed(21)
    c = (torch.randn(cfg.hidden_size, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
    emb = model.w["embedding"]
    emb0 = emb.clone()
    emb += c
    c_hat = c.float() / c.float().norm()
    routers = [layer["block_sparse_moe.router.layer"] for layer in model.w["layers"]]
    base = [r.clone() for r in routers]
    shares = []
    inner = model_module.route_add_rmsnorm

    def tapped(*a, **kw):
        weights, ids, z = inner(*a, **kw)
        shares.append(torch.isin(ids, hot).float().mean())
        return weights, ids, z

    def prefill(beta, timed=False):
        for r, b in zip(routers, base):
            rr = b.clone()
            rr[hot] = (rr[hot].float() + beta * c_hat).to(torch.bfloat16)
            r.copy_(rr)
        shares.clear()
        engine.reset()
        torch.cuda.synchronize()
        t = time.perf_counter()
        engine.prefill()
        torch.cuda.synchronize()
        return time.perf_counter() - t

    model_module.route_add_rmsnorm = tapped
    try:
        lo, hi = 0.0, 4.0
        for _ in range(12):
            beta = (lo + hi) / 2
            prefill(beta)
            if float(shares[0]) < 0.48:
                lo = beta
            else:
                hi = beta
        beta = (lo + hi) / 2
        prefill(beta)
        share0, share_last = float(shares[0]), float(shares[-1])
    finally:
        model_module.route_add_rmsnorm = inner
    times = [prefill(beta) for _ in range(4)]
    for r, b in zip(routers, base):
        r.copy_(b)
    emb.copy_(emb0)
    return {"ms": min(times[1:]) * 1e3, "beta": beta, "hot": list(hot_ids), "hot_share_layer0": share0,
            "hot_share_last_layer": share_last}


def prefill_bench(args):
    """cfg 4: packed prefill on the 3B shape (one JSON line)."""
    import torch

    from litemoe_amd import experts, packed, synth
    from litemoe_amd.config import preset
    from litemoe_amd.engine import Request
    from litemoe_amd.ep import ExpertParallel
    from litemoe_amd.experts import HipFusedExperts
    from litemoe_amd.model import Granite
    from litemoe_amd.optimized import OptimizedEngine

    dev = torch.device("cuda:0")
    cfg = preset(args.model)
    w = synth.granite_weights(cfg, seed=0, device=dev, method="torch")
    lengths = synth.ragged_lengths(48, 64, 2048, 2)
    tokens = sum(lengths)
    ep = ExpertParallel(1, 0, tokens, cfg.hidden_size, cfg.num_experts_per_tok, torch.bfloat16, dev,
                        HipFusedExperts())
    model = Granite(cfg, w, ep, 4096)
    prompts = synth.prompts(48, lengths, cfg.vocab_size, 1)
    engine = OptimizedEngine(model, [Request(str(i), p, 2) for i, p in enumerate(prompts)], ignore_eos=True)
    times = []
    with torch.inference_mode():
        for _ in range(4):
            engine.reset()
            torch.cuda.synchronize()
            t = time.perf_counter()
            engine.prefill()
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t)
        elapsed = min(times[1:])
        log(f"prefill of {tokens} tokens: {elapsed * 1e3:.1f} ms")
        # The same prefill with RoPE and the KV store as their own pass after
        # the QKV projection (Granite.qkv_epilogue off).
        model.qkv_epilogue = False
        times = []
        for _ in range(3):
            engine.reset()
            torch.cuda.synchronize()
            t = time.perf_counter()
            engine.prefill()
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t)
        model.qkv_epilogue = True
        unfused_ms = min(times[1:]) * 1e3
        log(f"prefill, separate RoPE/KV pass: {unfused_ms:.1f} ms")
        skew = skewed_prefill(model, engine, cfg, dev)
        log(f"prefill with cfg 4's skewed router (layer-0 hot share {skew['hot_share_layer0']:.3f}): "
            f"{skew['ms']:.1f} ms")

        # The MoE and the attention of one layer at the same token counts.
        H, I, E, k = cfg.hidden_size, cfg.intermediate_size, cfg.num_local_experts, cfg.num_experts_per_tok
        gen = torch.Generator(device=dev).manual_seed(5)
        z = torch.randn(tokens, H, device=dev, generator=gen).to(torch.bfloat16)
        layer = model.w["layers"][0]
        rng = torch.Generator().manual_seed(6)
        uniform = torch.stack([torch.randperm(E, generator=rng)[:k] for _ in range(tokens)]).int().to(dev)
        hot = torch.full((E,), 0.5 / (E - 4))
        hot[:4] = 0.5 / 4
        skewed = torch.multinomial(hot.expand(tokens, E), k, replacement=False, generator=rng).int().to(dev)
        moe_flops = tokens * k * 6 * I * H
        moe = {}
        # the weights the prefill reads (the checkpoint layout; the packed copy serves decode)
        w13, w2 = layer["input_linear"], layer["output_linear"]
        for name, ids in (("uniform", uniform), ("hot4_50pct", skewed)):
            y = experts.moe_routes(z, w13, w2, ids)
            ms = hip_time(lambda: experts.moe_routes(z, w13, w2, ids, y=y), 5)
            moe[name] = {"ms_per_layer": round(ms, 3), "tflops": round(moe_flops / ms / 1e9, 1),
                         "frac": round(moe_flops / ms / 1e9 / BF16_PEAK_TFLOPS, 4)}
        hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, 64
        q = torch.randn(tokens, hq, d, device=dev, generator=gen).to(torch.bfloat16)
        kk = torch.randn(tokens, hkv, d, device=dev, generator=gen).to(torch.bfloat16)
        vv = torch.randn(tokens, hkv, d, device=dev, generator=gen).to(torch.bfloat16)
        ends = torch.tensor(lengths, dtype=torch.int32).cumsum(0, dtype=torch.int32)
        cu = torch.cat((ends.new_zeros(1), ends)).to(dev)
        ms = hip_time(lambda: packed.varlen_attention(q, kk, vv, cu, max(lengths), cfg.attention_multiplier), 5)
        attn_flops = sum(n * (n + 1) // 2 for n in lengths) * hq * 4 * d
        # The dense projections (lm_linear) beside torch's F.linear (hipBLASLt) on the same operands.
        from litemoe_amd.linear import linear_dense
        projections = {}
        for name, weight in (("qkv", layer["self_attn.qkv_proj"]), ("o_proj", layer["self_attn.o_proj"])):
            out = torch.empty(tokens, weight.shape[0], device=dev, dtype=torch.bfloat16)
            own = hip_time(lambda: linear_dense(z, weight, out=out), 5)
            blas = hip_time(lambda: torch.nn.functional.linear(z, weight), 5)
            flops = 2 * tokens * H * weight.shape[0]
            projections[name] = {"ms": round(own, 4), "frac": round(flops / own / 1e9 / BF16_PEAK_TFLOPS, 4),
                                 "hipblaslt_ms": round(blas, 4),
                                 "hipblaslt_frac": round(flops / blas / 1e9 / BF16_PEAK_TFLOPS, 4)}
        # QKV projection with RoPE + KV store in its epilogue against the projection then lm_rope_kv_write
        from litemoe_amd.linear import linear_rope_kv
        from litemoe_amd.rope import rope_kv_write
        wq = layer["self_attn.qkv_proj"]
        pos = torch.cat([torch.arange(n) for n in lengths]).to(dev)
        slots = torch.repeat_interleave(torch.arange(len(lengths)), torch.tensor(lengths)).to(dev)
        act = torch.ones(tokens, dtype=torch.bool, device=dev)
        qkv = torch.empty(tokens, wq.shape[0], device=dev, dtype=torch.bfloat16)

        def two_pass():
            linear_dense(z, wq, out=qkv)
            rope_kv_write(qkv[:, :hq * d].view(tokens, hq, d), qkv[:, hq * d:(hq + hkv) * d].view(tokens, hkv, d),
                          qkv[:, (hq + hkv) * d:].view(tokens, hkv, d), pos, act, model.cos_sin, engine.cache, 0,
                          slots=slots, write_k=True)

        fused = hip_time(lambda: linear_rope_kv(z, wq, hq, hkv, pos, act, model.cos_sin, engine.cache, 0, slots), 5)
        separate = hip_time(two_pass, 5)
        projections["qkv_rope_kv"] = {"ms": round(fused, 4), "two_pass_ms": round(separate, 4)}
    line = {
        "metric": "prefill tok/s, Granite-3B-shape bf16, cfg4 packed prefill",
        "value": round(tokens / (skew["ms"] * 1e-3), 1),
        "unit": "tok/s", "n_gpus": 1, "higher_is_better": True, "dtype": "bf16",
        "data": "synthetic: random-init bf16 weights (seed 0), prompt ids (seed 1), lengths U{64..2048} (seed 2); "
                "skew vector seed 21",
        "config": {"workload": f"cfg4 packed prefill: {args.model} shape, 48 prompts, {tokens} tokens, router "
                               f"skewed so 4 experts take ~half of the routes",
                   "tokens": tokens, "ms": round(skew["ms"], 2), "hot_experts": skew["hot"],
                   "beta": round(skew["beta"], 4), "hot_share_layer0": round(skew["hot_share_layer0"], 4),
                   "hot_share_last_layer": round(skew["hot_share_last_layer"], 4)},
        "uniform_router": {"tok_s": round(tokens / elapsed, 1), "ms": round(elapsed * 1e3, 2)},
        "separate_rope_kv_ms": round(unfused_ms, 2),
        "moe_mfma": {"flops_per_layer": moe_flops, "peak_tflops": BF16_PEAK_TFLOPS, **moe},
        "projections_mfma": projections,
        "attention_mfma": {"flops_per_layer": attn_flops, "ms_per_layer": round(ms, 3),
                           "tflops": round(attn_flops / ms / 1e9, 1),
                           "frac": round(attn_flops / ms / 1e9 / BF16_PEAK_TFLOPS, 4)},
    }
    print(json.dumps(line), flush=True)


def flash_decode_bench(args):
    """cfg 5: decode attention, B=128, contexts U{1024..4096} (one JSON line)."""
    import numpy as np
    import torch

    from litemoe_amd.flash_decode import FlashDecode

    dev = torch.device("cuda:0")
    batch, hq, hkv, d, cap = 128, 24, 8, 64, 4096
    used_list = np.random.RandomState(3).randint(1024, 4097, size=batch)
    used = torch.tensor(used_list, dtype=torch.int32, device=dev)
    gen = torch.Generator(device=dev).manual_seed(8)
    k = torch.randn(batch, hkv, cap, d, device=dev, generator=gen).to(torch.bfloat16)
    v = torch.randn(batch, hkv, cap, d, device=dev, generator=gen).to(torch.bfloat16)
    q = torch.randn(batch, hq, 1, d, device=dev, generator=gen).to(torch.bfloat16)
    flash = FlashDecode(batch, hkv, hq // hkv, cap, dev, int(used_list.max()))
    zeros = torch.zeros(batch, dtype=torch.int64, device=dev)
    active = torch.ones(batch, dtype=torch.bool, device=dev)
    with torch.inference_mode():
        ms = hip_time(lambda: flash(q, k, v, zeros, active, 0.125, used=used), 20)
    kv_bytes = int(used_list.sum()) * hkv * d * 2 * 2 + batch * hq * d * 2 * 2
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    line = {
        "metric": "flash-decode GB/s, cfg5 (B=128, ctx U{1024..4096})", "value": round(gbs, 1), "unit": "GB/s",
        "n_gpus": 1, "higher_is_better": True, "dtype": "bf16", "data": "synthetic: KV N(0,1) (seed 8), contexts seed 3",
        "config": {"workload": "cfg5 decode attention, one layer", "batch": batch, "q_heads": hq, "kv_heads": hkv,
                   "capacity": cap, "splits": flash.splits},
        "us_per_layer": round(ms * 1e3, 2), "bytes_per_layer": kv_bytes,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4)},
    }
    print(json.dumps(line), flush=True)


def long_decode_bench(args):
    """cfg 5: decode steps at B=128 over ragged long contexts (one JSON line)."""
    import torch

    from litemoe_amd import synth
    from litemoe_amd.config import preset
    from litemoe_amd.engine import Request
    from litemoe_amd.ep import ExpertParallel
    from litemoe_amd.experts import HipFusedExperts
    from litemoe_amd.model import Granite
    from litemoe_amd.optimized import OptimizedEngine

    dev = torch.device("cuda:0")
    cfg = preset(args.model)
    batch, cap, steps, warmup = 128, 4096, 32, 5
    lengths = synth.ragged_lengths(batch, 1024, cap - 64, 3)
    w = synth.granite_weights(cfg, seed=0, device=dev, method="torch")
    ep = ExpertParallel(1, 0, batch, cfg.hidden_size, cfg.num_experts_per_tok, torch.bfloat16, dev,
                        HipFusedExperts())
    model = Granite(cfg, w, ep, cap)
    prompts = synth.prompts(batch, lengths, cfg.vocab_size, 1)
    requests = [Request(str(i), p, 48) for i, p in enumerate(prompts)]
    engine = OptimizedEngine(model, requests, mode="graph", ignore_eos=True, capacity=cap)
    with torch.inference_mode():
        engine.prepare_graph()
        engine.reset()
        t = time.perf_counter()
        engine.prefill()
        torch.cuda.synchronize()
        log(f"prefill of {sum(lengths)} tokens ({batch} prompts) in {time.perf_counter() - t:.2f}s")
        snapshot = {k: v.clone() for k, v in engine.state.items()}
        for _ in range(warmup):
            engine.graph.replay()
        torch.cuda.synchronize()
        for k, v in snapshot.items():
            engine.state[k].copy_(v)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            engine.graph.replay()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        assert bool(engine.state["active"].all())
    kv = sum(n + steps // 2 for n in lengths) * cfg.num_key_value_heads * 64 * 2 * 2 * cfg.num_hidden_layers
    line = {
        "metric": "decode tok/s, cfg5 (B=128, contexts U{1024..4032})", "value": round(batch * steps / elapsed, 1),
        "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(elapsed * 1e3 / steps, 4),
        "higher_is_better": True, "dtype": "bf16",
        "data": "synthetic: random-init bf16 weights (seed 0), prompt ids (seed 1), lengths seed 3",
        "config": {"workload": "cfg5 decode: granite-3b shape, batch 128, ragged prompts U{1024..4032}, capacity 4096, "
                               "one hipGraph per decode step", "batch": batch, "capacity": cap,
                   "mean_context": round(sum(lengths) / batch + steps / 2, 1)},
        "kv_bytes_per_step": kv,
    }
    print(json.dumps(line), flush=True)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cfg1_inputs():
    """cfg 1: x [16, 1024] N(0, 1) (seed 1), router [32, 1024], w13 [32, 1024,
    1024] and w2 [32, 1024, 512] N(0, 0.02) (seed 0), bf16."""
    from litemoe_amd import synth
    h, e, i, m = 1024, 32, 512, 16
    return (synth.normal_bf16((m, h), 1.0, synth.tensor_seed(1, 0)),
            synth.normal_bf16((e, h), 0.02, synth.tensor_seed(0, 0)),
            synth.normal_bf16((e, 2 * i, h), 0.02, synth.tensor_seed(0, 1)),
            synth.normal_bf16((e, h, i), 0.02, synth.tensor_seed(0, 2)))


def cfg1_moe_block_ms(threads, inputs, warmups=3, repeats=5):
    """cfg 1 timed directly: one 1B-shape MoE block (16 tokens, 32 experts
    top-8, intermediate 512) on LiteMoE's CPU path (router GEMM, topk,
    softmax, bf16 scales, per-row expert GEMMs, bf16 index_add combine):
    median of ``repeats`` after ``warmups``, in milliseconds."""
    import statistics

    import torch

    from oracle import ops
    torch.set_num_threads(threads)
    x, wr, w1, w2 = inputs
    k = 8

    def block():
        scores = ops.linear_rows(x, wr, True)
        top, ids = ops.select_topk(scores, k)
        scales = top.softmax(-1).to(torch.bfloat16).float()
        return ops.reference_experts(x, ids, scales, w1, w2, singleton=True)

    times = []
    for n in range(warmups + repeats):
        t0 = time.perf_counter()
        block()
        if n >= warmups:
            times.append(time.perf_counter() - t0)
    return statistics.median(times) * 1e3


def cpu_baseline(model, cfg, engine, state, layers, batch):
    """The CPU oracle's decode step (LiteMoE's torch CPU path restated) on
    ``layers`` of the model's layers, weights and the filled KV cache copied
    from the GPU, extrapolated to all layers; at 1 thread (the reference's
    own setting) and at every core this process may use. Plus cfg 1's MoE
    block timed directly."""
    import torch

    from oracle import granite as oracle
    all_cores = len(os.sched_getaffinity(0))

    def sample(n):
        sub = cfg.__class__(**{**cfg.to_dict(), "num_hidden_layers": n})
        w = {"embedding": model.w["embedding"].cpu(), "norm": model.w["norm"].cpu(),
             "head": model.w["head"].cpu(),
             "layers": [{k: v.cpu() for k, v in model.w["layers"][i].items()} for i in range(n)]}
        ref = oracle.Granite(sub, w, engine.capacity, fused=False)
        cache = oracle.Cache(sub, batch, engine.capacity, torch.bfloat16)
        if n:
            cache.k.copy_(engine.cache.k[:n].cpu())
            cache.v.copy_(engine.cache.v[:n].cpu())
        tokens, lengths = state["next"].cpu(), state["length"].cpu()
        valid = torch.ones(batch, dtype=torch.bool)
        ref.decode(tokens, lengths, valid, cache)  # warm-up
        times = []
        for _ in range(2):
            t0 = time.perf_counter()
            ref.decode(tokens, lengths, valid, cache)
            times.append(time.perf_counter() - t0)
        return min(times)

    steps = {}
    for threads in (1, all_cores):
        torch.set_num_threads(threads)
        t0, tl = sample(0), sample(layers)
        steps[threads] = (t0 + (tl - t0) * cfg.num_hidden_layers / layers, tl)
    inputs = cfg1_inputs()
    moe = {threads: cfg1_moe_block_ms(threads, inputs) for threads in (1, all_cores)}
    torch.set_num_threads(all_cores)
    step, tl = steps[all_cores]
    return dict(value=batch / step, unit="tok/s", cores=all_cores, kind="port",
                value_1_thread=batch / steps[1][0], cpu_model=cpu_model(),
                cfg1_moe_block_ms={"1_thread": round(moe[1], 2), f"{all_cores}_threads": round(moe[all_cores], 2)},
                sample=(f"CPU oracle decode step (LiteMoE torch CPU path: per-row bf16 GEMMs, masked attention, "
                        f"index_add combine) at batch {batch}, context {int(state['length'][0])}, timed on "
                        f"{layers} of {cfg.num_hidden_layers} layers plus embedding/head ({tl:.2f} s per step on "
                        f"{all_cores} threads, {steps[1][1]:.2f} s on 1) and extrapolated to "
                        f"{cfg.num_hidden_layers} layers ({step:.1f} s / {steps[1][0]:.1f} s per step); "
                        f"value on all {all_cores} cores of sched_getaffinity, value_1_thread at 1 thread "
                        f"(the reference's setting); cfg 1 MoE block (16 tokens, 1B shape) timed directly, "
                        f"median of 5 after 3 warm-ups"))


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if not 1 <= args.steps <= args.new_tokens - 1:
        print("--steps must be in [1, new_tokens - 1]", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.copy_probe:
        a = torch.full((256 << 20,), 1, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        log("copied 3 x 256 MiB")
        return

    if args.read_probe:
        a = torch.ones((2048, 65536), dtype=torch.bfloat16, device="cuda")
        for _ in range(3):
            a.sum(dim=1)
        torch.cuda.synchronize()
        log("read 3 x 256 MiB as 2048 rows of 128 KiB")
        return

    if args.prefill:
        return prefill_bench(args)
    if args.flash_decode:
        return flash_decode_bench(args)
    if args.long_decode:
        return long_decode_bench(args)

    from litemoe_amd import synth
    from litemoe_amd.config import preset
    from litemoe_amd.engine import Request
    from litemoe_amd.ep import ExpertParallel
    from litemoe_amd.experts import HipFusedExperts
    from litemoe_amd.model import Granite
    from litemoe_amd.optimized import OptimizedEngine, optimized_policy

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = preset(args.model)
    t = time.perf_counter()
    w = synth.granite_weights(cfg, seed=0, device=dev, method="torch")
    torch.cuda.synchronize()
    log(f"weights {args.model} generated in {time.perf_counter() - t:.1f}s")
    ep = ExpertParallel(1, 0, args.batch, cfg.hidden_size, cfg.num_experts_per_tok, torch.bfloat16, dev,
                        HipFusedExperts())
    model = Granite(cfg, w, ep, 4096)
    model.chain_combine = args.chained
    prompts = synth.prompts(args.batch, args.prompt, cfg.vocab_size, 1)
    requests = [Request(str(i), p, args.new_tokens) for i, p in enumerate(prompts)]
    if args.roofline_only:
        with torch.inference_mode():
            roof = moe_roofline(model, cfg, args.batch, args.roofline_reps)
        log(f"gate_up {roof['gate_up_us']:.1f} us/launch, fused MoE {roof['fused_us']:.1f} us/layer")
        print(json.dumps({k: (round(v, 3) if isinstance(v, float) else v) for k, v in roof.items()}), flush=True)
        return
    engine = OptimizedEngine(model, requests, mode="graph-async", ignore_eos=True)
    with torch.inference_mode():
        t = time.perf_counter()
        engine.prepare_graph()
        torch.cuda.synchronize()
        log(f"decode step captured in {time.perf_counter() - t:.1f}s (capacity {engine.capacity})")
        engine.reset()
        t = time.perf_counter()
        engine.prefill()
        torch.cuda.synchronize()
        log(f"prefill of {args.batch}x{args.prompt} tokens in {time.perf_counter() - t:.2f}s")
        snapshot = {k: v.clone() for k, v in engine.state.items()}
        for _ in range(args.warmup):
            engine.graph.replay()
        torch.cuda.synchronize()
        for k, v in snapshot.items():
            engine.state[k].copy_(v)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            engine.graph.replay()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        assert bool(engine.state["active"].all() or args.steps == args.new_tokens - 1)
        log(f"timed {args.steps} decode steps in {elapsed:.3f}s")
        value = args.batch * args.steps / elapsed

        roof = moe_roofline(model, cfg, args.batch, args.roofline_reps)
        log(f"gate_up {roof['gate_up_us']:.1f} us/launch, fused MoE {roof['fused_us']:.1f} us/layer")
        attention = decode_attention_rate(engine, cfg, args.roofline_reps)
        log(f"decode attention {attention['us_per_layer']:.1f} us/layer at mean context {attention['mean_context']}")

        engine_tps = None
        if not args.no_engine:
            _, metrics = engine.generate()
            engine_tps = metrics["decode_tps"]
            log(f"Engine.generate decode_tps {engine_tps:.1f}")

        cpu = None
        if not args.no_cpu_baseline:
            for k, v in snapshot.items():
                engine.state[k].copy_(v)
            with optimized_policy(engine):
                engine.prefill()
            torch.cuda.synchronize()
            cpu = cpu_baseline(model, cfg, engine, snapshot, args.cpu_layers, args.batch)
            log(f"cpu baseline {cpu['value']:.2f} tok/s on {cpu['cores']} threads, "
                f"{cpu['value_1_thread']:.3f} tok/s on 1 ({cpu['cpu_model']}); cfg1 MoE {cpu['cfg1_moe_block_ms']}")

    gate_gbs = roof["gate_up_bytes"] / (roof["gate_up_us"] * 1e-6) / 1e9
    fused_gbs = roof["fused_bytes"] / (roof["fused_us"] * 1e-6) / 1e9
    headline = args.model == "granite-3b" and args.batch == 64  # the profiled configuration
    name = {"granite-3b": "cfg3", "granite-1b": "cfg2"}.get(args.model, args.model)
    line = {
        "metric": METRIC if headline else f"decode tok/s, {args.model} shape bf16 bs={args.batch}",
        "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(elapsed * 1e3 / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random-init bf16 weights N(0,0.02) (torch generator, seed 0), random prompt ids (seed 1)",
        "config": {"workload": (f"{name} decode: {args.model} shape ({cfg.num_hidden_layers} layers, hidden "
                                f"{cfg.hidden_size}, {cfg.num_attention_heads}/{cfg.num_key_value_heads} heads, "
                                f"{cfg.num_local_experts} experts top-{cfg.num_experts_per_tok}, intermediate "
                                f"{cfg.intermediate_size}), batch {args.batch}, prompt {args.prompt}, "
                                f"{args.new_tokens} new tokens, greedy, one hipGraph per decode step"),
                   "global_batch": args.batch, "seq_len": args.prompt, "new_tokens": args.new_tokens,
                   "capacity": engine.capacity, "parallelism": "single GPU",
                   "timed_contexts": [args.prompt, args.prompt + args.steps - 1],
                   "mean_context": round(args.prompt + (args.steps - 1) / 2, 1)},
        "roofline": {"bound": "hbm", "kernel": "gate_up_scan_kernel (lm_moe_gate_up_packed)",
                     "achieved": round(gate_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gate_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("gate_up_scan_kernel.granite3b_b64_decode.txt") if headline else None,
                     "traffic_source": ("rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE of this kernel, calibrated on a copy, "
                                        "read from profiles/gate_up_scan_kernel.granite3b_b64_decode.txt (not measured "
                                        "in this run)") if headline else None,
                     "bytes_per_launch": int(roof["gate_up_bytes"]), "us_per_launch": round(roof["gate_up_us"], 2),
                     "active_experts": roof["active"]},
        "fused_moe": {"achieved": round(fused_gbs, 1), "unit": "GB/s", "frac": round(fused_gbs / HBM_PEAK_GBS, 4),
                      "us_per_layer": round(roof["fused_us"], 2), "bytes_per_layer": int(roof["fused_bytes"]),
                      "launches": ("gate/up; down with the combine and the residual add (the next norm is "
                                   "formed by the QKV projection)") if roof["chained"] else
                                  "gate/up; down; combine with the residual add and the next norm"},
        "decode_attention": attention,
        "engine_decode_tps": None if engine_tps is None else round(engine_tps, 1),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
