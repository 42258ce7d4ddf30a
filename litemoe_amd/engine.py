"""Requests, GPU-owned greedy state, the decode step and the generate loop.

Mirrors litemoe/engine.py:15-221 for one GPU: the same state tensors
(``next``, ``length``, ``generated``, ``budget``, ``present``, ``active``),
the same ``emit [B, 3] = (token, index, valid)`` snapshot, the same capacity
rule and metrics (``decode_tps = decode_tokens / decode_s``). Prefill is the
packed ragged path (litemoe/packed.py:19-36), run in chunks of at most
``prefill_tokens`` tokens.
"""
import math
import time
from dataclasses import dataclass

import torch

from .cache import KVCache
from .execution import OutputRing, capture_decode
from .packed import packed_prefill_logits


@dataclass
class Request:
    request_id: str
    prompt: list
    budget: int


def prepare_batch(model, tokens):
    """Grow the expert dispatch capacity for ``tokens`` rows (batch.py:7-11)."""
    model.ep.capacity = max(model.ep.capacity, tokens)
    model.ep.prepare(tokens)


class Engine:
    cache_type = KVCache
    prefill_tokens = 1 << 17

    def __init__(self, model, requests, world=1, rank=0, mode="eager", ignore_eos=False, poll=1,
                 capacity=None, host_process=None):
        if world != 1 or rank != 0:
            raise ValueError("This build runs one engine per GPU (world == 1)")
        self.model, self.world, self.rank = model, world, rank
        self.device, self.dtype = model.w["embedding"].device, model.w["embedding"].dtype
        if poll < 1 or mode not in ("eager", "graph", "graph-async"):
            raise ValueError("Invalid execution mode or polling period")
        if any(type(r.budget) is not int or r.budget < 0 for r in requests):
            raise ValueError("Output budgets must be nonnegative integers")
        if len({r.request_id for r in requests}) != len(requests):
            raise ValueError("Request ids must be unique")
        self.empty = {r.request_id: [] for r in requests if r.budget == 0}
        self.requests = [r for r in requests if r.budget]
        cfg = model.cfg
        if any(not r.prompt or any(type(t) is not int or not 0 <= t < cfg.vocab_size for t in r.prompt)
               for r in self.requests):
            raise ValueError("Each prompt must contain valid vocabulary ids")
        required = max((len(r.prompt) + r.budget - 1 for r in self.requests), default=1)
        if required > min(4096, cfg.max_position_embeddings):
            raise ValueError("Request exceeds the model context limit")
        cap = capacity or (2 ** math.ceil(math.log2(required)) if mode != "eager" else required)
        if cap < required or cap > min(4096, cfg.max_position_embeddings):
            raise ValueError("Insufficient/unsupported KV capacity")
        if cap > model.capacity:
            raise ValueError("KV capacity exceeds the model's RoPE table")
        self.capacity = cap
        self.batch = len(self.requests)
        self.local = self.requests
        self.mode, self.ignore_eos, self.poll = mode, ignore_eos, poll
        self.host_process = host_process
        self.graph = None
        if not self.requests:
            return
        if self.device.type != "cuda":
            raise ValueError("This engine runs on the GPU path only")
        if mode != "eager" and not model.ep.backend.graph_safe:
            raise ValueError("Full Decode Graph requires a graph-safe expert backend")
        self.cache = self.cache_type(cfg, self.batch, cap, self.device, self.dtype)
        self.state = {name: torch.zeros(self.batch, dtype=dtype, device=self.device) for name, dtype in (
            ("next", torch.int64), ("length", torch.int64), ("generated", torch.int64),
            ("budget", torch.int64), ("present", torch.bool), ("active", torch.bool),
        )}
        self.emit = torch.zeros(self.batch, 3, dtype=torch.int64, device=self.device)
        eos = cfg.eos_token_id
        self.eos = torch.tensor(eos if isinstance(eos, list) else ([] if eos is None else [eos]),
                                device=self.device, dtype=torch.int64)
        prepare_batch(model, self.batch)
        self.reset()

    def reset(self):
        self.cache.reset()
        for value in self.state.values():
            value.zero_()
        budgets = torch.tensor([r.budget for r in self.local], dtype=torch.int64)
        self.state["budget"].copy_(budgets)
        self.state["present"].fill_(True)
        self.emit.zero_()

    def is_eos(self, token):
        if self.eos.numel() == 0:
            return torch.zeros_like(token, dtype=torch.bool)
        return (token[:, None] == self.eos[None, :]).any(-1)

    def decode_step(self):
        s = self.state
        if getattr(self.model, "decode_lean", False) and self.model.greedy_supported():
            # Lean decode: the step's set-up and its argmax/state update run
            # as one kernel each around the layers (same tokens and state).
            self.model.greedy_step(s, self.emit, self.eos, self.ignore_eos, self.cache)
            return
        valid = s["active"].clone()
        positions = torch.where(valid, s["length"], 0)[:, None]
        logits = self.model.forward(s["next"][:, None], positions, valid[:, None], self.cache)
        candidate = logits[:, 0].argmax(-1)
        self.emit[:, 0].copy_(candidate)
        self.emit[:, 1].copy_(s["generated"])
        self.emit[:, 2].copy_(valid)
        s["length"].add_(valid)
        s["generated"].add_(valid)
        s["next"].copy_(torch.where(valid, candidate, s["next"]))
        done = s["generated"] >= s["budget"]
        if not self.ignore_eos:
            done = done | self.is_eos(candidate)
        s["active"].copy_(valid & ~done)

    def prepare_graph(self):
        if self.mode == "eager" or self.graph is not None or not self.requests:
            return
        if self.model.trace is not None:
            raise ValueError("Trace/count collection must be disabled during capture/timing")

        def warm_state():
            self.reset()
            self.state["active"].copy_(self.state["present"])
            self.state["budget"].fill_(2)

        self.graph = capture_decode(self.decode_step, warm_state)
        self.reset()

    def synchronize(self):
        torch.cuda.synchronize(self.device)

    def stopped(self):
        return self.state["active"].sum(dtype=torch.int64).item() == 0

    def prefill_logits(self, prompts):
        """Last-position logits of every prompt, packed in token-bounded chunks."""
        out, start = [], 0
        while start < len(prompts):
            end, tokens = start, 0
            while end < len(prompts) and (end == start or tokens + len(prompts[end]) <= self.prefill_tokens):
                tokens += len(prompts[end])
                end += 1
            prepare_batch(self.model, tokens)
            out.append(packed_prefill_logits(self.model, prompts[start:end], self.cache, start))
            start = end
        return out[0] if len(out) == 1 else torch.cat(out)

    def prefill(self):
        first = self.prefill_logits([r.prompt for r in self.local])[:, 0].argmax(-1)
        s = self.state
        s["next"].copy_(first)
        s["length"].copy_(torch.tensor([len(r.prompt) for r in self.local], device=self.device))
        s["generated"].copy_(s["present"])
        active = s["present"] & (s["budget"] > 1)
        if not self.ignore_eos:
            active &= ~self.is_eos(first)
        s["active"].copy_(active)

    @torch.inference_mode()
    def generate(self, step_events=None):
        if not self.requests:
            return self.empty, dict(prefill_s=0.0, decode_s=0.0, e2e_s=0.0, input_tokens=0, output_tokens=0,
                                    decode_tokens=0, decode_tps=None, e2e_tps=None)
        self.prepare_graph()
        self.reset()
        outputs = [[] for _ in self.local]

        def consume(rows):
            for slot, (token, index, valid) in enumerate(rows):
                if valid:
                    if slot >= len(outputs) or index != len(outputs[slot]):
                        raise RuntimeError("Lost, duplicated or reordered output snapshot")
                    outputs[slot].append(token)
                    if self.host_process:
                        self.host_process(outputs[slot])

        ring = OutputRing(self.emit, consume, self.mode == "graph-async")
        self.synchronize()
        start = time.perf_counter()
        self.prefill()
        s = self.state
        self.emit[:, 0].copy_(s["next"])
        self.emit[:, 1].zero_()
        self.emit[:, 2].copy_(s["present"])
        consume(self.emit.cpu().tolist())  # first tokens are published before decode
        self.synchronize()
        prefill_end = time.perf_counter()
        hard_limit = max(r.budget for r in self.requests) - 1
        done = not self.ignore_eos and self.stopped()
        for n in range(hard_limit):
            if done:
                break
            if step_events is not None:
                begin, finish = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                begin.record()
            if self.graph:
                self.graph.replay()
            else:
                self.decode_step()
            if step_events is not None:
                finish.record()
                step_events.append((begin, finish))
            ring.publish(n)
            if not self.ignore_eos and (n + 1) % self.poll == 0:
                done = self.stopped()
        ring.drain()
        self.synchronize()
        end = time.perf_counter()
        p, d, e = prefill_end - start, end - prefill_end, end - start
        inp = sum(len(r.prompt) for r in self.local)
        out = sum(map(len, outputs))
        dec = sum(max(len(o) - 1, 0) for o in outputs)
        result = {r.request_id: o for r, o in zip(self.local, outputs)}
        result.update(self.empty)
        return result, dict(prefill_s=p, decode_s=d, e2e_s=e, input_tokens=inp, output_tokens=out,
                            decode_tokens=dec, decode_tps=dec / d if dec else None, e2e_tps=out / e,
                            capacity=self.capacity)
