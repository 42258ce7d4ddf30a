"""Requests, the GPU-resident greedy state, the decode step and the generate loop.

The public surface is the reference's (litemoe/engine.py:15-221): ``Request``,
``Engine(model, requests, world, rank, mode, ignore_eos, poll, capacity,
host_process)``, ``decode_step()``, ``prefill()``, ``prepare_graph()``,
``stopped()`` and ``generate()`` with the same metrics keys, the same
``emit [B, 3] = (token, index, valid)`` snapshot and its ordering check.
The engine runs one GPU (world 1). What differs is how a step runs:

* the decode step's set-up and its argmax/state update are one kernel each
  (``lm_decode_prologue``, ``lm_greedy_epilogue``) around the layers; a step
  on a model without that path runs its forward and then the same epilogue
  kernel, so both share one state update;
* in ``graph-async`` mode the epilogue also writes each step's emit rows
  straight into a pinned host ring (:class:`OutputRing`), so a replay is the
  only launch per step;
* when to stop is read from the delivered snapshots (a row ends when its
  outputs reach its budget or its last token is a stop id), so the loop
  polls without a device synchronisation;
* ``prefill`` runs one ``forward(..., slot=j)`` per request as the
  reference's plain engine does (engine.py:128-148); the model executes each
  on its packed kernels. The batched engines (``batch.BatchPrefillEngine``,
  ``optimized.OptimizedEngine``) prefill every request in one padded or
  packed call instead.
"""
import math
import time
from dataclasses import dataclass

import torch

from .cache import KVCache
from .execution import OutputRing, capture_decode
from .step import greedy_epilogue

CONTEXT_LIMIT = 4096
STATE_FIELDS = (("next", torch.int64), ("length", torch.int64), ("generated", torch.int64),
                ("budget", torch.int64), ("present", torch.bool), ("active", torch.bool))


@dataclass
class Request:
    request_id: str
    prompt: list
    budget: int


@dataclass
class _Plan:
    """Validated requests of one engine and the KV capacity they need."""
    live: list
    empty: dict
    capacity: int


def plan_requests(requests, cfg, mode, capacity, rope_rows):
    """Check a request list the way litemoe/engine.py:33-51 does (same
    messages) and choose the KV capacity: the longest prompt plus its budget,
    rounded up to a power of two for the graph modes."""
    if any(type(r.budget) is not int or r.budget < 0 for r in requests):
        raise ValueError("Output budgets must be nonnegative integers")
    if len({r.request_id for r in requests}) != len(requests):
        raise ValueError("Request ids must be unique")
    live = [r for r in requests if r.budget]
    empty = {r.request_id: [] for r in requests if not r.budget}
    vocab = cfg.vocab_size
    for r in live:
        if not r.prompt or any(type(t) is not int or not 0 <= t < vocab for t in r.prompt):
            raise ValueError("Each prompt must contain valid vocabulary ids")
    limit = min(CONTEXT_LIMIT, cfg.max_position_embeddings)
    need = max((len(r.prompt) + r.budget - 1 for r in live), default=1)
    if need > limit:
        raise ValueError("Request exceeds the model context limit")
    if not capacity:  # None or 0 chooses, as the reference's `capacity or ...` (engine.py:47)
        capacity = need if mode == "eager" else 1 << math.ceil(math.log2(need))
    if not need <= capacity <= limit:
        raise ValueError("Insufficient/unsupported KV capacity")
    if capacity > rope_rows:
        raise ValueError("KV capacity exceeds the model's RoPE table")
    return _Plan(live, empty, capacity)


class Engine:
    cache_type = KVCache
    ring_depth = 4

    def __init__(self, model, requests, world=1, rank=0, mode="eager", ignore_eos=False, poll=1,
                 capacity=None, host_process=None):
        if world != 1 or rank != 0:
            raise ValueError("This build runs one engine per GPU (world == 1)")
        if poll < 1 or mode not in ("eager", "graph", "graph-async"):
            raise ValueError("Invalid execution mode or polling period")
        self.model, self.world, self.rank = model, world, rank
        embedding = model.w["embedding"]
        self.device, self.dtype = embedding.device, embedding.dtype
        plan = plan_requests(requests, model.cfg, mode, capacity, model.capacity)
        self.requests, self.empty, self.capacity = plan.live, plan.empty, plan.capacity
        self.local = self.requests
        self.batch = len(self.requests)
        # prefill rounds: the longest prompt of each group of `world` requests
        # (litemoe/engine.py:69); with one rank, each request's prompt length
        self.rounds = [len(r.prompt) for r in self.requests]
        self.mode, self.ignore_eos, self.poll, self.host_process = mode, ignore_eos, poll, host_process
        self.graph = None
        self.ring = None
        if not self.requests:
            return
        if self.device.type != "cuda":
            raise ValueError("This engine runs on the GPU path only")
        if mode != "eager" and not model.ep.backend.graph_safe:
            raise ValueError("Full Decode Graph requires a graph-safe expert backend")
        cfg = model.cfg
        self.cache = self.cache_type(cfg, self.batch, self.capacity, self.device, self.dtype)
        self.state = {name: torch.zeros(self.batch, dtype=dtype, device=self.device)
                      for name, dtype in STATE_FIELDS}
        self.emit = torch.zeros(self.batch, 3, dtype=torch.int64, device=self.device)
        eos = cfg.eos_token_id
        self.eos_ids = [] if eos is None else list(eos) if isinstance(eos, (list, tuple)) else [eos]
        self.eos = torch.tensor(self.eos_ids, device=self.device, dtype=torch.int64)
        self.budgets = [r.budget for r in self.requests]
        self._consumer = None
        self.ring = OutputRing(self.emit, self._consume, mode == "graph-async", self.ring_depth)
        model.ep.capacity = max(model.ep.capacity, self.batch)
        model.ep.prepare(self.batch)
        self.reset()

    # -- state ---------------------------------------------------------------
    def reset(self):
        self.cache.reset()
        s = self.state
        for value in s.values():
            value.zero_()
        s["budget"].copy_(torch.tensor(self.budgets, dtype=torch.int64))
        s["present"].fill_(True)
        self.emit.zero_()

    def is_eos(self, token):
        if not self.eos_ids:
            return torch.zeros_like(token, dtype=torch.bool)
        return torch.isin(token, self.eos)

    def stopped(self):
        """Whether no row is active (reads the device state; the generate
        loop decides from the delivered snapshots instead)."""
        return not bool(self.state["active"].any())

    # -- one decode step ---------------------------------------------------------
    def decode_step(self):
        s = self.state
        ring = self.ring if self.ring is not None and self.ring.asynchronous else None
        if getattr(self.model, "decode_lean", False) and self.model.greedy_supported():
            self.model.greedy_step(s, self.emit, self.eos, self.ignore_eos, self.cache, ring=ring)
            return
        # Any other model: the torch prologue, its forward (which divides by
        # logits_scaling itself, so the epilogue scales by 1: an exact
        # product), and the shared epilogue kernel for argmax and state.
        valid = s["active"].clone()
        positions = torch.where(valid, s["length"], 0)[:, None]
        logits = self.model.forward(s["next"][:, None], positions, valid[:, None], self.cache)[:, 0]
        greedy_epilogue(logits, 1.0, valid, s, self.emit, self.eos, self.ignore_eos)

    def prepare_graph(self):
        if self.mode == "eager" or self.graph is not None or not self.requests:
            return
        if self.model.trace is not None:
            raise ValueError("Trace/count collection must be disabled during capture/timing")

        def steady():  # every present row active, one token of budget left
            self.reset()
            self.state["active"].copy_(self.state["present"])
            self.state["budget"].fill_(2)

        self.graph = capture_decode(self.decode_step, steady)
        self.reset()

    def synchronize(self):
        torch.cuda.synchronize(self.device)

    # -- prefill -------------------------------------------------------------------
    def start_rows(self, first):
        """State for the first decode step after a prefill that chose the
        tokens ``first``: lengths, one output generated, and each row active
        unless its budget is 1 or (without ignore_eos) the token stops it
        (litemoe/batch.py:57-64)."""
        s = self.state
        s["next"].copy_(first)
        s["length"].copy_(torch.tensor([len(r.prompt) for r in self.local], device=self.device))
        s["generated"].copy_(s["present"])
        keep = s["present"] & (s["budget"] > 1)
        if not self.ignore_eos:
            keep &= ~self.is_eos(first)
        s["active"].copy_(keep)

    def prefill(self):
        """One forward per request into its own cache row, as
        litemoe/engine.py:128-148 (``slot=j``, the last prompt position)."""
        firsts = []
        for j, length in enumerate(self.rounds):
            prompt = self.local[j].prompt
            tokens = torch.tensor([prompt], device=self.device)
            pos = torch.arange(len(prompt), device=self.device)[None, :]
            valid = torch.ones_like(tokens, dtype=torch.bool)
            logits = self.model.forward(tokens, pos, valid, self.cache, slot=j, last=len(prompt) - 1,
                                        communication_tokens=length)
            firsts.append(logits[0, 0].argmax(-1))
        self.start_rows(torch.stack(firsts))

    # -- generation ------------------------------------------------------------------
    def _consume(self, rows):
        self._consumer(rows)

    @torch.inference_mode()
    def generate(self, step_events=None):
        if not self.requests:
            return self.empty, dict(prefill_s=0.0, decode_s=0.0, e2e_s=0.0, input_tokens=0, output_tokens=0,
                                    decode_tokens=0, decode_tps=None, e2e_tps=None)
        self.prepare_graph()
        self.reset()
        outputs = [[] for _ in self.local]
        open_rows = set(range(self.batch))  # rows whose snapshots may still add tokens
        stops = set(self.eos_ids)

        def consume(rows):
            for slot, (token, index, valid) in enumerate(rows):
                if not valid:
                    continue
                out = outputs[slot] if slot < len(outputs) else None
                if out is None or index != len(out):
                    raise RuntimeError("Lost, duplicated or reordered output snapshot")
                out.append(token)
                if self.host_process:
                    self.host_process(out)
                if len(out) >= self.budgets[slot] or (not self.ignore_eos and token in stops):
                    open_rows.discard(slot)

        self._consumer = consume
        self.synchronize()
        start = time.perf_counter()
        self.prefill()
        s = self.state
        self.emit[:, 0].copy_(s["next"])
        self.emit[:, 1].zero_()
        self.emit[:, 2].copy_(s["present"])
        consume(self.emit.cpu().tolist())  # the first tokens, before any decode step
        self.synchronize()
        prefill_end = time.perf_counter()
        self.ring.start()
        steps = max(self.budgets) - 1
        for n in range(steps):
            if not self.ignore_eos and n % self.poll == 0:
                # Snapshots arrive up to ring_depth - 1 steps late in the
                # asynchronous mode; no replay is queued once every row is
                # known closed, or once no open row has budget left for it
                # (step n emits each row's output n + 2).
                if not open_rows or n + 2 > max(self.budgets[j] for j in open_rows):
                    break
            if step_events is not None:
                begin, finish = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                begin.record()
            if self.graph is not None:
                self.graph.replay()
            else:
                self.decode_step()
            if step_events is not None:
                finish.record()
                step_events.append((begin, finish))
            self.ring.publish(n)
        self.ring.drain()
        self.synchronize()
        end = time.perf_counter()
        prefill_s, decode_s, e2e_s = prefill_end - start, end - prefill_end, end - start
        input_tokens = sum(len(r.prompt) for r in self.local)
        output_tokens = sum(map(len, outputs))
        decode_tokens = sum(max(len(o) - 1, 0) for o in outputs)
        result = {r.request_id: o for r, o in zip(self.local, outputs)}
        result.update(self.empty)
        return result, dict(prefill_s=prefill_s, decode_s=decode_s, e2e_s=e2e_s, input_tokens=input_tokens,
                            output_tokens=output_tokens, decode_tokens=decode_tokens,
                            decode_tps=decode_tokens / decode_s if decode_tokens else None,
                            e2e_tps=output_tokens / e2e_s, capacity=self.capacity)
